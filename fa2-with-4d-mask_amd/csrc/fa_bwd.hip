// FlashAttention-2 backward for gfx950 (MI355X) with optional 4D keep-mask and
// 4D fp32 score: the kernels around the dK/dV kernel (fa_bwd_kv.hip) and the
// dQ kernels (fa_bwd_dq.hip).  Restates the maths of the reference's TileLang
// backward (python/fa2.py:142-426):
//
//   preprocess   Delta[b,h,i] = sum_d O*dO (fp32)          (python/fa2.py:142-179)
//                + the backward's LSE, rows with no kept key, a zeroed fp32
//                dQ accumulator where dQ partials are added
//   dq           dQ without a dS workspace: one workgroup per (128 query
//                rows, head, batch) recomputes S, P, dP and dS per key tile
//                (with a mask only the prepared lists' live tiles) and
//                forms dQ = dS K in registers
//   convert      fp32 accumulators (dQ partials, dK/dV slabs of a head-group
//                split) -> bf16/fp16 outputs, slabs summed in a fixed order.
#include "fa_common.h"
#include "fa_kernels.h"

namespace fa {
namespace {

template <typename T>
__device__ __forceinline__ u32x2 pack4(float x0, float x1, float x2, float x3) {
  typedef T T4 __attribute__((ext_vector_type(4)));
  T4 v;
  v[0] = (T)x0; v[1] = (T)x1; v[2] = (T)x2; v[3] = (T)x3;
  return __builtin_bit_cast(u32x2, v);
}

template <typename T>
__device__ __forceinline__ float to_f(T x) { return (float)x; }

// ---------------------------------------------------------------------------
// preprocess: Delta, the backward's LSE, dead-row flags, zeroed dQ accumulator
// rows
// ---------------------------------------------------------------------------
// Whether query row q of (b, h) keeps at least one key: j < Tk, j <= q when
// causal, and the mask bit (the prepared bits are zero past Tk).  Only asked
// for rows whose LSE is +inf, so a serial scan of the row's words is fine.
__device__ bool row_keeps_a_key(const PreArgs& a, int b, int h, int q) {
  if (!a.mws) return true;   // no mask: key 0 is kept (j <= q holds for j = 0)
  const int pm = mask_plane(a.ml, b, h);
  const uint32_t* w = (const uint32_t*)(a.mws + a.ml.bits + pm * a.ml.pbits) + (int64_t)q * a.ml.wk;
  const int nw = a.is_causal ? min(q / 32 + 1, a.ml.nk32) : a.ml.nk32;
  for (int i = 0; i < nw; ++i) {
    uint32_t x = w[i];
    if (a.is_causal && i == q / 32 && (q & 31) != 31) x &= (2u << (q & 31)) - 1u;
    if (x) return true;
  }
  return false;
}

template <typename T, int D>
__global__ __launch_bounds__(256) void preprocess_kernel(const PreArgs a) {
  constexpr int CH = D / 8;            // 16-byte chunks per row
  constexpr int CPT = CH / 4;          // chunks per thread (4 threads per row)
  const int h = blockIdx.y, b = blockIdx.z;
  const int r = threadIdx.x >> 2, part = threadIdx.x & 3;
  const int q = blockIdx.x * 64 + r;
  float acc = 0.f;
  if (q < a.Tq) {
    const T* op = (const T*)a.o + b * a.osb + (int64_t)q * a.ost + h * a.osh;
    const T* dp = (const T*)a.dout + b * a.dsb + (int64_t)q * a.dst + h * a.dsh;
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = part + 4 * u;
      const auto ov = as_vec8<T>(gload16(op + c * 8));
      const auto dv = as_vec8<T>(gload16(dp + c * 8));
#pragma unroll
      for (int t = 0; t < 8; ++t) acc = fmaf(to_f<T>(ov[t]), to_f<T>(dv[t]), acc);
    }
    if (a.olo) {
      // O's rounding residual from the forward (mask or score): O to about
      // 16 significant bits
      const T* lp = (const T*)a.olo + b * a.olsb + (int64_t)q * a.olst + h * a.olsh;
#pragma unroll
      for (int u = 0; u < CPT; ++u) {
        const int c = part + 4 * u;
        const auto lv = as_vec8<T>(gload16(lp + c * 8));
        const auto dv = as_vec8<T>(gload16(dp + c * 8));
#pragma unroll
        for (int t = 0; t < 8; ++t) acc = fmaf(to_f<T>(lv[t]), to_f<T>(dv[t]), acc);
      }
    }
  }
  acc += __shfl_xor(acc, 1);
  acc += __shfl_xor(acc, 2);
  if (q < a.Tq) {
    if (a.dq_accum) {
      float* z = a.dq_accum + (((int64_t)b * a.Hq + h) * a.Tq + q) * D + part * (D / 4);
#pragma unroll
      for (int u = 0; u < D / 16; ++u) *(f32x4*)(z + 4 * u) = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (part == 0) {
      const int64_t ri = ((int64_t)b * a.Hq + h) * a.Tq + q;
      // LSE = +inf: every kept logit of the row is -inf.  Either the row
      // keeps no key (eager: dQ row 0, masked_fill's backward) or its kept
      // keys all carry a -inf score (eager: the softmax row is NaN, and so
      // are the dQ row and the dK rows of those keys).  The backward kernels
      // take P = exp2(s c - LSE_b) and select dropped entries to 0: LSE_b =
      // +inf gives P = 0 everywhere, LSE_b = -inf gives NaN on exactly the
      // kept entries (s = -inf there).  dV of the kv-head is NaN either way.
      const float lse = a.lse[ri];
      const bool dead = lse == kPosInf;
      a.delta[ri] = dead ? 0.f : acc;
      a.lse_b[ri] = dead ? (row_keeps_a_key(a, b, h, q) ? kNegInf : kPosInf) : lse;
      if (dead) a.dead[b * a.Hk + h / a.G] = 1;
    }
  }
}

// ---------------------------------------------------------------------------
// deterministic dQ
// ---------------------------------------------------------------------------
constexpr int kDqBM = 128;   // query rows per workgroup (4 waves x 32)
constexpr int kDqBN = 64;    // keys per tile

// Without a mask or a score two workgroups share a CU (256 registers per
// wave, a dozen spilled): one wave's MFMAs overlap the other's softmax and
// dS work, which a lone wave issues in sequence (H: 2.53 -> 1.82 ms, causal
// 1.47 -> 0.97).  The masked and score instances (P and dS in two parts)
// keep one wave per SIMD: 256 registers would spill about a hundred.
template <typename T, int D, bool CAUSAL, bool MASK, bool SCORE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu((MASK || SCORE) ? 1 : 2, (MASK || SCORE) ? 1 : 2)))
void dq_kernel(const BwdArgs a) {
  using V8 = typename Vec8<T>::type;
  static_assert(D <= 128, "head dim 256 recomputes dQ in fa_wide.hip");
  constexpr int BM = kDqBM, BN = kDqBN;
  constexpr int NKB = BN / 32;   // 32-key blocks per tile
  constexpr int DS = D / 16, NB = D / 32, CH = D / 8;
  constexpr int KS = D + 40;   // K: row-wise and transposed reads
  constexpr int VS = D + 8;    // V: row-wise reads only
  constexpr int KT = BN * KS, VT = BN * VS;
  constexpr int U = BN * CH / 256;
  constexpr int OS = D + 8;
  static_assert(4 * 32 * OS <= 2 * (KT + VT), "dQ staging fits");
  constexpr bool PREC = MASK || SCORE;
  __shared__ __attribute__((aligned(16))) T smem[2 * (KT + VT)];

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

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hf = lane >> 5;
  const int q0 = qt * BM, q0w = q0 + wave * 32;
  const int qrow = q0w + l32;
  const int Tq = a.Tq, Tk = a.Tk;
  const float c2 = a.scale_log2, scale = a.scale;

  const T* __restrict__ qp = (const T*)a.q + b * a.qsb + h * a.qsh;
  const T* __restrict__ dp = (const T*)a.dout + b * a.dsb + h * a.dsh;
  const T* __restrict__ kp = (const T*)a.k + b * a.ksb + kvh * a.ksh;
  const T* __restrict__ vp = (const T*)a.v + b * a.vsb + kvh * a.vsh;

  V8 qf[DS], dof[DS];
  float lse_q = kPosInf, delta_q = 0.f;
  if (qrow < Tq) {
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      qf[ds] = as_vec8<T>(gload16(qp + (int64_t)qrow * a.qst + ds * 16 + hf * 8));
      dof[ds] = as_vec8<T>(gload16(dp + (int64_t)qrow * a.dst + ds * 16 + hf * 8));
    }
    lse_q = a.lse[((int64_t)b * a.Hq + h) * Tq + qrow];
    delta_q = a.delta[((int64_t)b * a.Hq + h) * Tq + qrow];
  } else {
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      qf[ds] = as_vec8<T>(u32x4{0, 0, 0, 0});
      dof[ds] = as_vec8<T>(u32x4{0, 0, 0, 0});
    }
  }
  const int qrow_c = min(qrow, Tq - 1);
  const float* srow = nullptr;
  if constexpr (SCORE) srow = a.score + b * a.ssb + h * a.ssh + (int64_t)qrow_c * a.ssq;

  // Key tiles: 0 .. ntiles-1, or with a mask the live 64-key tiles of the
  // prepared list of this block's 256-row unit (the forward's lists; causality
  // folded in; bit 31: every entry kept), and the keep bits of this lane's
  // row from the prepared bit array
  static_assert(!MASK || (BN == kFwdKeys && kFwdRows % BM == 0), "prepared-mask list shape");
  const int32_t* flist = nullptr;
  const uint32_t* mbits = nullptr;
  if constexpr (MASK) {
    const int pm = mask_plane(a.ml, b, h);
    flist = (const int32_t*)(a.mws + a.ml.lfwd + pm * a.ml.plfwd) + (int64_t)(q0 / kFwdRows) * (1 + a.ml.nft);
    mbits = (const uint32_t*)(a.mws + a.ml.bits + pm * a.ml.pbits) + (int64_t)qrow_c * a.ml.wk;
  }
  const int kv_end = CAUSAL ? min(Tk, q0 + BM) : Tk;
  const int ntiles = MASK ? flist[0] : (kv_end + BN - 1) / BN;
  // list entries of positions j, j+1, j+2 (the next tile's loads are issued a
  // tile ahead, its entry read a tile before that)
  auto entry = [&](int j) __attribute__((always_inline)) -> int32_t {
    if constexpr (MASK) return j < ntiles ? flist[1 + j] : 0;
    else return j;
  };
  int32_t e_cur = entry(0), e_nx = entry(1);

  u32x4 kreg[U], vreg[U];
  // Keys past Tk are loaded from key Tk-1 (unconditional loads): their P is
  // masked to 0, so they contribute nothing.
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = tid + u * 256;
      const int r = idx / CH, c = idx % CH;
      const int kk = min(k0 + r, Tk - 1);
      kreg[u] = gload16(kp + (int64_t)kk * a.kst + c * 8);
      vreg[u] = gload16(vp + (int64_t)kk * a.vst + c * 8);
    }
  };
  auto store_tile = [&](int buf) {
    T* ks = smem + buf * (KT + VT);
    T* vs = ks + KT;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = tid + u * 256;
      const int r = idx / CH, c = idx % CH;
      lds_write16(ks + r * KS + c * 8, kreg[u]);
      lds_write16(vs + r * VS + c * 8, vreg[u]);
    }
  };

  f32x16 qacc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) qacc[nb] = f32x16{};
  const int tr_row = 4 * hf + ((lane >> 2) & 3);
  const int tr_col = ((lane >> 4) & 1) * 16 + (lane & 3) * 4;

  load_tile((e_cur & 0x7fffffff) * BN);
  store_tile(0);
  __syncthreads();
  for (int j = 0; j < ntiles; ++j) {
    const int k0 = (e_cur & 0x7fffffff) * BN;
    const bool more = j + 1 < ntiles;
    if (more) load_tile((e_nx & 0x7fffffff) * BN);
    const int32_t e_nx2 = entry(j + 2);
    const T* ks = smem + (j & 1) * (KT + VT);
    const T* vs = ks + KT;
    const bool active = !CAUSAL || (k0 <= q0w + 31);
    if (active) {
      f32x16 sacc[NKB], pacc[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        sacc[kb] = f32x16{};
        pacc[kb] = f32x16{};
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
          const u32x4 kx = lds_read16(ks + (kb * 32 + l32) * KS + ds * 16 + hf * 8);
          sacc[kb] = mfma32(as_vec8<T>(kx), qf[ds], sacc[kb]);
          const u32x4 vx = lds_read16(vs + (kb * 32 + l32) * VS + ds * 16 + hf * 8);
          pacc[kb] = mfma32(as_vec8<T>(vx), dof[ds], pacc[kb]);
        }
      }
      // (with a mask: keep words of this tile's two 32-key blocks)
      uint32_t mw[MASK ? NKB : 1] = {};
      if constexpr (MASK) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) mw[kb] = (k0 >> 5) + kb < a.ml.nk32 ? mbits[(k0 >> 5) + kb] : 0u;
      }
      const bool edge = (MASK && e_cur >= 0) || (k0 + BN > Tk) || (CAUSAL && k0 + BN - 1 > q0w);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int kk = k0 + kb * 32 + gi * 8 + hf * 4;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int i = gi * 4 + t;
            const int kx = kk + t;
            float s = sacc[kb][i];
            if constexpr (SCORE) s += kx < Tk ? srow[kx] : 0.f;
            if (a.zero_scale) s = 0.f;
            float p = exp2_fast(fmaf(s, c2, -lse_q));
            if (edge) {
              bool keep = kx < Tk;
              if constexpr (CAUSAL) keep = keep && kx <= qrow;
              if constexpr (MASK) keep = keep && ((mw[kb] >> (kx & 31)) & 1u) != 0;
              p = keep ? p : 0.f;
            }
            sacc[kb][i] = p * (pacc[kb][i] - delta_q) * scale;
          }
        }
      // dQ^T += K^T dS^T: A = K^T via transpose reads, B = dS^T from registers.
      // With a mask or a score dS enters in two 16-bit parts (the rounded value
      // and its rounding residual), as in the dK/dV and dQ-from-dS kernels.
#pragma unroll
      for (int kk2 = 0; kk2 < 2 * NKB; ++kk2) {
        const int kb = kk2 >> 1, c = kk2 & 1;
        V8 dsb, dsl;
        if constexpr (PREC) {
          u32x4 wh, wl;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            uint32_t h2, l2;
            split2<T>(sacc[kb][8 * c + 2 * k], sacc[kb][8 * c + 2 * k + 1], &h2, &l2);
            wh[k] = h2;
            wl[k] = l2;
          }
          dsb = as_vec8<T>(wh);
          dsl = as_vec8<T>(wl);
        } else {
          dsb = pack8<T>(sacc[kb][8 * c + 0], sacc[kb][8 * c + 1], sacc[kb][8 * c + 2], sacc[kb][8 * c + 3],
                         sacc[kb][8 * c + 4], sacc[kb][8 * c + 5], sacc[kb][8 * c + 6], sacc[kb][8 * c + 7]);
        }
        const int row = kb * 32 + 16 * c + tr_row;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int col = nb * 32 + tr_col;
          const V8 ak = cat_tr<T>(lds_read_tr(ks + row * KS + col), lds_read_tr(ks + (row + 8) * KS + col));
          qacc[nb] = mfma32(ak, dsb, qacc[nb]);
          if constexpr (PREC) qacc[nb] = mfma32(ak, dsl, qacc[nb]);
        }
      }
    }
    if (more) store_tile((j + 1) & 1);
    __syncthreads();
    e_cur = e_nx;
    e_nx = e_nx2;
  }

  T* os = smem + wave * 32 * OS;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int gi = 0; gi < 4; ++gi)
      lds_write8(os + l32 * OS + nb * 32 + gi * 8 + hf * 4,
                 pack4<T>(qacc[nb][gi * 4 + 0], qacc[nb][gi * 4 + 1], qacc[nb][gi * 4 + 2], qacc[nb][gi * 4 + 3]));
  __syncthreads();
  T* dqp = (T*)a.dq + b * a.dqsb + h * a.dqsh;
#pragma unroll
  for (int u = 0; u < 32 * CH / 64; ++u) {
    const int idx = lane + u * 64;
    const int r = idx / CH, c = idx % CH;
    const int qr = q0w + r;
    if (qr < Tq) gstore16(dqp + (int64_t)qr * a.dqst + c * 8, lds_read16(os + r * OS + c * 8));
  }
}

// ---------------------------------------------------------------------------
// fp32 accumulator -> dtype
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void convert_kernel(const CvtArgs a) {
  const int64_t nchunk = (int64_t)a.B * a.T * a.H * (a.D / 8);
  const int cpr = a.D / 8;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nchunk; i += (int64_t)gridDim.x * 256) {
    const int c = (int)(i % cpr);
    int64_t rest = i / cpr;
    const int hh = (int)(rest % a.H); rest /= a.H;
    const int t = (int)(rest % a.T);
    const int bb = (int)(rest / a.T);
    const float* s = a.src + bb * a.src_sb + (int64_t)t * a.src_st + (int64_t)hh * a.src_sh + c * 8;
    f32x4 x0 = *(const f32x4*)s, x1 = *(const f32x4*)(s + 4);
    for (int k = 1; k < a.nsplit; ++k) {  // fixed summation order: deterministic
      x0 += *(const f32x4*)(s + k * a.split_stride);
      x1 += *(const f32x4*)(s + k * a.split_stride + 4);
    }
    const auto v = pack8<T>(x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]);
    T* d = (T*)a.dst + bb * a.sb + (int64_t)t * a.st + hh * a.sh + c * 8;
    gstore16(d, as_u32x4<T>(v));
  }
}

template <typename T, int D, bool CAUSAL>
hipError_t launch_dq_t(const BwdArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.B * a.Hq * a.nqt)), block(256);
  const bool m = a.mask != nullptr, sc = a.score != nullptr;
  if (m && sc) hipLaunchKernelGGL((dq_kernel<T, D, CAUSAL, true, true>), grid, block, 0, s, a);
  else if (m) hipLaunchKernelGGL((dq_kernel<T, D, CAUSAL, true, false>), grid, block, 0, s, a);
  else if (sc) hipLaunchKernelGGL((dq_kernel<T, D, CAUSAL, false, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((dq_kernel<T, D, CAUSAL, false, false>), grid, block, 0, s, a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_pre_t(const PreArgs& a, int D, hipStream_t s) {
  const dim3 grid((unsigned)((a.Tq + 63) / 64), (unsigned)a.Hq, (unsigned)a.B), block(256);
  if (D == 128) hipLaunchKernelGGL((preprocess_kernel<T, 128>), grid, block, 0, s, a);
  else if (D == 64) hipLaunchKernelGGL((preprocess_kernel<T, 64>), grid, block, 0, s, a);
  else if (D == 256) hipLaunchKernelGGL((preprocess_kernel<T, 256>), grid, block, 0, s, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace

int dq_block_rows() { return kDqBM; }

hipError_t launch_preprocess(const PreArgs& a, int D, int dtype, hipStream_t s) {
  return dtype == 0 ? launch_pre_t<bf16>(a, D, s) : launch_pre_t<f16>(a, D, s);
}

hipError_t launch_bwd_dq(const BwdArgs& a, int D, int dtype, bool causal, hipStream_t s) {
  if (dtype == 0) {
    if (D == 128) return causal ? launch_dq_t<bf16, 128, true>(a, s) : launch_dq_t<bf16, 128, false>(a, s);
    if (D == 64) return causal ? launch_dq_t<bf16, 64, true>(a, s) : launch_dq_t<bf16, 64, false>(a, s);
  } else {
    if (D == 128) return causal ? launch_dq_t<f16, 128, true>(a, s) : launch_dq_t<f16, 128, false>(a, s);
    if (D == 64) return causal ? launch_dq_t<f16, 64, true>(a, s) : launch_dq_t<f16, 64, false>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_convert(const CvtArgs& a, int dtype, hipStream_t s) {
  const int64_t nchunk = (int64_t)a.B * a.T * a.H * (a.D / 8);
  int64_t blocks = (nchunk + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  if (dtype == 0) hipLaunchKernelGGL((convert_kernel<bf16>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  else hipLaunchKernelGGL((convert_kernel<f16>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace fa
