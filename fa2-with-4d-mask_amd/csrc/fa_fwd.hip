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
//   M(i): S(i) = K(i) Q^T and O += V(i-1)^T P(i-1)      (MFMA phase)
//   V(i): softmax of S(i) -> P(i), lazy rescale of O    (VALU phase)
// Waves w and w+4 share a SIMD, so while one issues MFMAs the other issues
// VALU work; a workgroup barrier separates the phases.  K/V tiles are
// double-buffered in LDS and prefetched into registers two phases ahead; the
// barrier waits only for LDS traffic, never for those loads.
//
// The running maximum is only moved when a tile's maximum exceeds it by more
// than 2^8 (exact: O and l are rescaled consistently; p <= 256), which removes
// the accumulator rescale from almost every tile.
#include "fa_common.h"
#include "fa_kernels.h"

namespace fa {
namespace {

constexpr int kWaves = 8;               // two groups of four
constexpr int kBM = kWaves * 32;        // query rows per workgroup
constexpr int kBN = 64;                 // keys per tile
constexpr int kThreads = kWaves * 64;
constexpr float kRescaleLog2 = 8.0f;

__device__ __forceinline__ uint32_t load_mask4(const uint8_t* row, int kk, int Tk, bool vec) {
  if (vec && kk + 4 <= Tk) return *(const uint32_t*)(row + kk);
  uint32_t r = 0;
#pragma unroll
  for (int t = 0; t < 4; ++t)
    if (kk + t < Tk) r |= (uint32_t)(row[kk + t] != 0) << (8 * t);
  return r;
}

__device__ __forceinline__ f32x4 load_score4(const float* row, int kk, int Tk, bool vec) {
  if (vec && kk + 4 <= Tk) return *(const f32x4*)(row + kk);
  f32x4 r;
#pragma unroll
  for (int t = 0; t < 4; ++t) r[t] = (kk + t < Tk) ? row[kk + t] : 0.f;
  return r;
}

template <typename T>
__device__ __forceinline__ u32x2 pack4(float x0, float x1, float x2, float x3) {
  typedef T T4 __attribute__((ext_vector_type(4)));
  T4 v;
  v[0] = (T)x0; v[1] = (T)x1; v[2] = (T)x2; v[3] = (T)x3;
  return __builtin_bit_cast(u32x2, v);
}

// Workgroup barrier that waits for this wave's LDS traffic only: prefetch loads
// to registers stay in flight across it.
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
  // Padded row strides (elements): K rows are read 16 rows x 16 B at a time
  // (stride = 4 dwords mod 64 banks), V rows by the transpose read 4 rows x
  // 64 B at a time (stride = 16 dwords mod 64 banks): both conflict-free, and
  // every LDS address is a per-lane base plus an immediate offset.
  constexpr int KS = D + 8, VS = D + 32;
  constexpr int KT = BN * KS, VT = BN * VS;  // elements of one K / V tile
  constexpr int U = BN * CH / kThreads;      // 16-byte chunks per thread per tile
  static_assert(U >= 1 && BN * CH % kThreads == 0, "tile split");
  constexpr int OS = D + 8;                  // epilogue O staging stride
  static_assert(kWaves * 32 * OS <= 2 * (KT + VT), "O staging fits in the K/V buffers");
  __shared__ __attribute__((aligned(16))) T smem[2 * (KT + VT)];
  T* const kbuf = smem;           // [2][KT]
  T* const vbuf = smem + 2 * KT;  // [2][VT]

  // ---- which (batch, head, query tile) -------------------------------------
  // Logical order (b, kv-head, [query tile descending, head in group]); with
  // the XCD remap each XCD works on few kv-heads (K/V stay in its L2) and
  // causal work is dispatched longest-first.
  const int nblk = a.B * a.Hq * a.nqt;
  const int W = xcd_remap(blockIdx.x, nblk);
  const int per_kv = a.G * a.nqt;
  const int bk = W / per_kv;
  const int rem = W - bk * per_kv;
  const int qt_rev = rem / a.G;
  const int g = rem - qt_rev * a.G;
  const int qt = a.nqt - 1 - qt_rev;
  const int b = bk / a.Hk, kvh = bk - b * a.Hk;
  const int h = kvh * a.G + g;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = tid >> 6, grp = wave >> 2;
  const int l32 = lane & 31, hf = lane >> 5;
  const int q0 = qt * BM, q0w = q0 + wave * 32;
  const int qrow = q0w + l32;
  const int Tq = a.Tq, Tk = a.Tk;

  const T* __restrict__ qp = (const T*)a.q + b * a.qsb + h * a.qsh;
  const T* __restrict__ kp = (const T*)a.k + b * a.ksb + kvh * a.ksh;
  const T* __restrict__ vp = (const T*)a.v + b * a.vsb + kvh * a.vsh;

  // ---- Q fragment: lane holds Q[qrow][16 ds + 8 hf + 0..7] -------------------
  V8 qf[DS];
  {
    const uint32_t neg = a.qsign < 0.f ? 0x80008000u : 0u;
    const T* src = qp + (int64_t)min(qrow, Tq - 1) * a.qst + hf * 8;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      u32x4 x = gload16(src + ds * 16);
      x ^= neg;
      qf[ds] = as_vec8<T>(x);
    }
  }

  const int kv_end = CAUSAL ? min(Tk, q0 + BM) : Tk;
  const int nt = (kv_end + BN - 1) / BN;                       // tiles of the workgroup
  const int nt_w = CAUSAL ? min(nt, (min(Tk, q0w + 32) + BN - 1) / BN) : nt;  // tiles of this wave

  // Keys past Tk are loaded from key Tk-1 (unconditional loads, no zero fill):
  // the edge path masks them to -inf, so P = 0 there and V stays finite.
  // Full tiles use per-thread row pointers advanced by a uniform tile offset.
  u32x4 kreg[U], vreg[U];
  static_assert(kThreads % CH == 0, "chunk u of a thread is kThreads/CH rows below chunk 0");
  const T* const kthr = kp + (int64_t)(tid / CH) * a.kst + (tid % CH) * 8;
  const T* const vthr = vp + (int64_t)(tid / CH) * a.vst + (tid % CH) * 8;
  const int64_t ktile = (int64_t)BN * a.kst, vtile = (int64_t)BN * a.vst;
  const int64_t kstep = (int64_t)(kThreads / CH) * a.kst, vstep = (int64_t)(kThreads / CH) * a.vst;
  auto load_k = [&](int j) {
    if ((j + 1) * BN <= Tk) {
#pragma unroll
      for (int u = 0; u < U; ++u) kreg[u] = gload16(kthr + (j * ktile + u * kstep));
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int idx = tid + u * kThreads;
        const int key = min(j * BN + idx / CH, Tk - 1);
        kreg[u] = gload16(kp + (int64_t)key * a.kst + (idx % CH) * 8);
      }
    }
  };
  auto load_v = [&](int j) {
    if ((j + 1) * BN <= Tk) {
#pragma unroll
      for (int u = 0; u < U; ++u) vreg[u] = gload16(vthr + (j * vtile + u * vstep));
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int idx = tid + u * kThreads;
        const int key = min(j * BN + idx / CH, Tk - 1);
        vreg[u] = gload16(vp + (int64_t)key * a.vst + (idx % CH) * 8);
      }
    }
  };
  auto store_k = [&](int j) {
    T* ks = kbuf + (j & 1) * KT;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = tid + u * kThreads;
      lds_write16(ks + (idx / CH) * KS + (idx % CH) * 8, kreg[u]);
    }
  };
  auto store_v = [&](int j) {
    T* vs = vbuf + (j & 1) * VT;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = tid + u * kThreads;
      lds_write16(vs + (idx / CH) * VS + (idx % CH) * 8, vreg[u]);
    }
  };

  const int qrow_c = min(qrow, Tq - 1);  // clamped row for mask/score reads
  const uint8_t* mrow = nullptr;
  const float* srow = nullptr;
  if constexpr (MASK) mrow = a.mask + b * a.msb + h * a.msh + (int64_t)qrow_c * a.msq;
  if constexpr (SCORE) srow = a.score + b * a.ssb + h * a.ssh + (int64_t)qrow_c * a.ssq;
  const bool mvec = a.mask_vec != 0, svec = a.score_vec != 0;
  const float c2 = a.scale_log2;
  const int tr_row = 4 * hf + ((lane >> 2) & 3);
  const int tr_col = ((lane >> 4) & 1) * 16 + (lane & 3) * 4;

  f32x16 oacc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) oacc[nb] = f32x16{};
  f32x16 sacc[2] = {f32x16{}, f32x16{}};
  V8 pk[4];                        // P(i) packed for the next M step
  uint32_t mreg[MASK ? 8 : 1];     // mask bytes of the tile in flight
  f32x4 sreg[SCORE ? 8 : 1];       // score of the tile in flight
  float m_run = kNegInf, l_run = 0.f;

  // prologue: K(0) in LDS, K(1) and V(0) in flight
  load_k(0);
  store_k(0);
  if (nt > 1) load_k(1);
  load_v(0);
  lds_barrier();

  const int nph = 2 * nt + 2;
  for (int ph = 0; ph < nph; ++ph) {
    const int st = ph - grp;  // this wave's step
    if (st >= 0 && st <= 2 * nt) {
      const int i = st >> 1;
      if ((st & 1) == 0) {
        // ---- M(i): S(i) = K(i) Q^T and O += V(i-1)^T P(i-1) ----------------------
        const bool do_s = i < nt_w;
        const bool do_pv = i >= 1 && i - 1 < nt_w;
        const T* ks = kbuf + (i & 1) * KT;
        const T* vs = vbuf + ((i - 1) & 1) * VT;
        if (do_s) {
          if constexpr (MASK || SCORE) {
            const int k0 = i * BN;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
              for (int gi = 0; gi < 4; ++gi) {
                const int kk = k0 + kb * 32 + gi * 8 + hf * 4;
                if constexpr (MASK) mreg[kb * 4 + gi] = load_mask4(mrow, kk, Tk, mvec);
                if constexpr (SCORE) sreg[kb * 4 + gi] = load_score4(srow, kk, Tk, svec);
              }
          }
          sacc[0] = f32x16{};
          sacc[1] = f32x16{};
        }
        if (do_s && do_pv) {
          // The two independent chains interleaved, S op t = (kb = t%2, ds = t/2),
          // PV op t = (kk = t/NB, nb = t%NB); operands are read from LDS three
          // op-pairs ahead of their MFMAs so the LDS latency hides behind them.
          constexpr int NOP = 2 * DS;   // == 4 * NB
          constexpr int AHEAD = 3;
          auto rd_s = [&](int t) -> u32x4 {
            return lds_read16(ks + ((t & 1) * 32 + l32) * KS + (t >> 1) * 16 + hf * 8);
          };
          auto rd_pv = [&](int t) -> V8 {
            const int kk = t / NB, nb = t % NB;
            const int row = (kk >> 1) * 32 + 16 * (kk & 1) + tr_row;
            const int col = nb * 32 + tr_col;
            return cat_tr<T>(lds_read_tr(vs + row * VS + col), lds_read_tr(vs + (row + 8) * VS + col));
          };
          u32x4 kq[AHEAD];
          V8 vq[AHEAD];
#pragma unroll
          for (int t = 0; t < AHEAD; ++t) {
            kq[t] = rd_s(t);
            vq[t] = rd_pv(t);
          }
          __builtin_amdgcn_sched_group_barrier(0x100, 3 * AHEAD, 0);
#pragma unroll
          for (int t = 0; t < NOP; ++t) {
            sacc[t & 1] = mfma32(as_vec8<T>(kq[t % AHEAD]), qf[t >> 1], sacc[t & 1]);
            oacc[t % NB] = mfma32(vq[t % AHEAD], pk[t / NB], oacc[t % NB]);
            if (t + AHEAD < NOP) {
              kq[t % AHEAD] = rd_s(t + AHEAD);
              vq[t % AHEAD] = rd_pv(t + AHEAD);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            if (t + AHEAD < NOP) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
          }
        } else if (do_s) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int ds = 0; ds < DS; ++ds) {
              const u32x4 kx = lds_read16(ks + (kb * 32 + l32) * KS + ds * 16 + hf * 8);
              sacc[kb] = mfma32(as_vec8<T>(kx), qf[ds], sacc[kb]);
            }
        } else if (do_pv) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            const int row = (kk >> 1) * 32 + 16 * (kk & 1) + tr_row;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              const int col = nb * 32 + tr_col;
              const s16x4 lo = lds_read_tr(vs + row * VS + col);
              const s16x4 hi = lds_read_tr(vs + (row + 8) * VS + col);
              oacc[nb] = mfma32(cat_tr<T>(lo, hi), pk[kk], oacc[nb]);
            }
          }
        }
      } else if (i < nt_w) {
        // ---- V(i): softmax of S(i) -> P(i) -----------------------------------------
        // lane's entry (kb, e) is key 64 i + 32 kb + 8 (e/4) + 4 hf + e%4 of row qrow
        const int k0 = i * BN;
        if constexpr (SCORE) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int gi = 0; gi < 4; ++gi)
#pragma unroll
              for (int t = 0; t < 4; ++t)
                sacc[kb][gi * 4 + t] = fmaf(a.qsign, sreg[kb * 4 + gi][t], sacc[kb][gi * 4 + t]);
        }
        const bool edge = MASK || a.zero_scale || (k0 + BN > Tk) || (CAUSAL && k0 + BN - 1 > q0w);
        if (edge) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
              const int kk = k0 + kb * 32 + gi * 8 + hf * 4;
              uint32_t mb = 0x01010101u;
              if constexpr (MASK) mb = mreg[kb * 4 + gi];
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                const int key = kk + t;
                bool keep = key < Tk;
                if constexpr (CAUSAL) keep = keep && (key <= qrow);
                if constexpr (MASK) keep = keep && (((mb >> (8 * t)) & 0xffu) != 0);
                const float sv = sacc[kb][gi * 4 + t];
                sacc[kb][gi * 4 + t] = keep ? (a.zero_scale ? 0.f : sv) : kNegInf;
              }
            }
        }
        float mx = kNegInf;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sacc[kb][e]);
        mx = half_max(mx);
        const float m_tile = mx * c2;
        if (wave_any(m_tile > m_run + kRescaleLog2)) {
          const float m_new = fmaxf(m_run, m_tile);
          const float alpha = (m_run == kNegInf) ? 0.f : exp2_fast(m_run - m_new);
          l_run *= alpha;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int e = 0; e < 16; ++e) oacc[nb][e] *= alpha;
          m_run = m_new;
        }
        const float mneg = (m_run == kNegInf) ? 0.f : -m_run;
        float lsum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const float p = exp2_fast(fmaf(sacc[kb][e], c2, mneg));
            sacc[kb][e] = p;
            lsum += p;
          }
        l_run += lsum;
        // key slot t of k-step kk (= 2 kb + c) <-> key 32 kb + 16 c + 4 hf + t%4 + 8 (t/4)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int kb = kk >> 1, c = kk & 1;
          pk[kk] = pack8<T>(sacc[kb][8 * c + 0], sacc[kb][8 * c + 1], sacc[kb][8 * c + 2], sacc[kb][8 * c + 3],
                            sacc[kb][8 * c + 4], sacc[kb][8 * c + 5], sacc[kb][8 * c + 6], sacc[kb][8 * c + 7]);
        }
      }
    }
    if (ph & 1) {
      // odd phase 2j+1: K(j+1) and V(j) to LDS, then prefetch K(j+2) and V(j+1)
      const int j = ph >> 1;
      if (j + 1 < nt) store_k(j + 1);
      if (j < nt) store_v(j);
      if (j + 2 < nt) load_k(j + 2);
      if (j + 1 < nt) load_v(j + 1);
    }
    lds_barrier();
  }

  // ---- epilogue: O = acc / l (NaN for a row with no kept key), LSE ----------------
  const float l_tot = half_sum(l_run);
  const float inv = 1.0f / l_tot;
  T* os = smem + wave * 32 * OS;  // wave-private staging, K/V buffers are free now
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
#pragma unroll
  for (int u = 0; u < 32 * CH / 64; ++u) {
    const int idx = lane + u * 64;
    const int r = idx / CH, c = idx % CH;
    const int qr = q0w + r;
    if (qr < Tq) gstore16(op + (int64_t)qr * a.ost + c * 8, lds_read16(os + r * OS + c * 8));
  }
  if (hf == 0 && qrow < Tq)
    a.lse[((int64_t)b * a.Hq + h) * Tq + qrow] = (l_tot > 0.f) ? m_run + log2_fast(l_tot) : kPosInf;
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
