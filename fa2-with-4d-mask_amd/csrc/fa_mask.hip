// Prepared mask for the gfx950 attention kernels: one pass over the bool
// keep-mask (the reference streams it per tile inside every kernel,
// python/fa2.py:107-114, 261-280) producing
//   * the mask as bits, row-major (forward, dQ) and transposed (dK/dV), so the
//     attention kernels read 1 bit per (row, key) instead of 1 byte;
//   * the state of every 32x32 block (no kept entry / some / all);
//   * per kernel work unit, the list of tiles that hold a kept entry (with
//     causality folded in), so dead tiles cost neither loads nor MFMAs.
// Layout: MaskLayout (fa_kernels.h).
#include "fa_common.h"
#include "fa_kernels.h"

namespace fa {
namespace {

constexpr int kRows = 32;     // rows per workgroup of the bits kernel (one row word)
constexpr int kKeys = 1024;   // keys per workgroup (1 KB of each row)

// Bit j of the result = (byte j of x) != 0, for the 4 bytes of x.
__device__ __forceinline__ uint32_t nz4(uint32_t x) {
  uint32_t t = x | (x >> 4);
  t |= t >> 2;
  t |= t >> 1;
  t &= 0x01010101u;                      // bit 8 j = byte j != 0
  return ((t * 0x01020408u) >> 24) & 0xfu;  // gathered into bits 0..3 (no carries)
}

// 32x32 bit transpose across each 32-lane half of a wave: lane r holds word r
// of the matrix (bit c = column c); afterwards lane c holds column c (bit r =
// row r).  Five block-swap stages (16, 8, 4, 2, 1): the lane with bit j clear
// takes its partner's low j-bit groups into its high ones, the partner the
// reverse; partner values come from ds_swizzle (xor j within 32 lanes).
template <int J>
__device__ __forceinline__ uint32_t transpose_stage(uint32_t a, bool hi, uint32_t m) {
  const uint32_t p = (uint32_t)__builtin_amdgcn_ds_swizzle((int)a, (J << 10) | 0x1f);
  const uint32_t sh = hi ? (p >> J) : (p << J);
  const uint32_t keep = hi ? ~m : m;   // bits of a that stay
  return (a & keep) | (sh & ~keep);
}
__device__ __forceinline__ uint32_t transpose32(uint32_t a, int l32) {
  a = transpose_stage<16>(a, (l32 & 16) != 0, 0x0000ffffu);
  a = transpose_stage<8>(a, (l32 & 8) != 0, 0x00ff00ffu);
  a = transpose_stage<4>(a, (l32 & 4) != 0, 0x0f0f0f0fu);
  a = transpose_stage<2>(a, (l32 & 2) != 0, 0x33333333u);
  a = transpose_stage<1>(a, (l32 & 1) != 0, 0x55555555u);
  return a;
}

// Grid (key chunk of 1024, row block of 32, plane).  Wave w reads rows
// 8 w .. 8 w + 7 of the block, one instruction per row: lane l the 16 bytes
// of keys 16 l .. 16 l + 15 of the chunk, so that each load instruction
// covers one whole 1 KB row segment; lane pairs (2 c, 2 c + 1) join their 16
// bits into the row word of key block c.  Every word written (bits
// row-major, bitsT per key block) lands in full 128-byte lines.
// One (key chunk of 1024, row block of 32 rows from r0, plane pm) of the bits
// kernel below.
__device__ __forceinline__ void bits_block(const MaskArgs& a, uint32_t (&words)[kRows][kKeys / 32 + 1], int kc0,
                                           int r0, int pm) {
  const MaskLayout& ml = a.ml;
  const int tid = threadIdx.x;
  const int bb = pm / ml.Hm, hh = pm - bb * ml.Hm;
  const uint8_t* src = a.mask + bb * a.msb + hh * a.msh;
  const int Tq = a.Tq, Tk = a.Tk;
  uint32_t* bits = (uint32_t*)(a.ws + ml.bits + pm * ml.pbits);
  uint32_t* bitsT = (uint32_t*)(a.ws + ml.bitsT + pm * ml.pbitsT);
  uint8_t* blk = (uint8_t*)(a.ws + ml.blk + pm * ml.pblk);

  {
    const int wv = tid >> 6, l = tid & 63, k16 = kc0 + 16 * l;
    // all rows' bytes are loaded before any word is stored (the stores could
    // alias the mask as far as the compiler knows)
    const bool vec = a.vec16 && k16 + 16 <= Tk;
    u32x4 x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = r0 + 8 * wv + i;
      x[i] = u32x4{0, 0, 0, 0};
      if (vec && row < Tq) x[i] = *(const u32x4*)(src + row * a.msq + k16);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rl = 8 * wv + i, row = r0 + rl;
      uint32_t h = 0;
      if (vec) {
#pragma unroll
        for (int j = 0; j < 4; ++j) h |= nz4(x[i][j]) << (4 * j);
      } else if (row < Tq && k16 < Tk) {
        const uint8_t* p = src + row * a.msq + k16;
        const int n = min(16, Tk - k16);
        for (int j = 0; j < n; ++j) h |= (uint32_t)(p[j] != 0) << j;
      }
      // lane 2 c takes lane 2 c + 1's 16 bits (ds_swizzle xor 1 within 32 lanes)
      const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_swizzle((int)h, (1 << 10) | 0x1f);
      if ((l & 1) == 0) words[rl][l >> 1] = h | (hi << 16);
    }
  }
  __syncthreads();
  {
    // row-major words: thread t stores rows t/32 + 8 i, key block t%32
    const int c = tid & 31, wcol = kc0 / 32 + c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rl = (tid >> 5) + 8 * i, row = r0 + rl;
      if (row < Tq && wcol < ml.wk) bits[(int64_t)row * ml.wk + wcol] = words[rl][c];   // padding words are 0
    }
  }

  // transposed: each half-wave turns the 32 row words of one key block into
  // the 32 key words (bit r = row r0 + r), four passes of two blocks per wave;
  // the 32 keys of a key block fill one 128-byte line.  The block's state
  // comes from the same words by two ballots over the half-wave: some valid
  // key keeps some valid row (any), every valid key keeps every valid row
  // (all).
  const int s = r0 / 32;
  const int wv = tid >> 6, l32 = tid & 31, hw = (tid >> 5) & 1;
  const int nr = min(32, Tq - r0);
  const uint32_t vrows = nr >= 32 ? 0xffffffffu : ((1u << nr) - 1u);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int cb = wv * 8 + 2 * q + hw;   // key block within the chunk
    const uint32_t w = transpose32(words[l32][cb], l32) & vrows;
    const int kk = kc0 + 32 * cb + l32;
    const bool valid = kk < Tk;
    if (valid) bitsT[((int64_t)(kk >> 5) * ml.wq + s) * 32 + (kk & 31)] = w;
    const uint32_t any = (uint32_t)(__builtin_amdgcn_ballot_w64(valid && w != 0) >> (32 * hw));
    const uint32_t notall = (uint32_t)(__builtin_amdgcn_ballot_w64(valid && w != vrows) >> (32 * hw));
    const int kb = kc0 / 32 + cb;
    if (l32 == 0 && kb < ml.nk32) blk[(int64_t)s * ml.nk32 + kb] = any == 0 ? 0 : (notall == 0 ? 2 : 1);
  }
}

__global__ __launch_bounds__(256) void mask_bits_kernel(const MaskArgs a) {
  __shared__ uint32_t words[kRows][kKeys / 32 + 1];
  const MaskLayout& ml = a.ml;
  const int kc0 = blockIdx.x * kKeys;
  const int nrb = (a.Tq + kRows - 1) / kRows, np = ml.Bm * ml.Hm;
  // row blocks and planes with grid strides: the grid's y and z hold at most
  // 65535 (the loop bounds are uniform in the workgroup, and so its barriers)
  for (int pm = blockIdx.z; pm < np; pm += gridDim.z) {
    for (int rb = blockIdx.y; rb < nrb; rb += gridDim.y) {
      bits_block(a, words, kc0, rb * kRows, pm);
      __syncthreads();   // words is rewritten for the next (row block, plane)
    }
  }
}

// One wave per list; lanes test 64 candidates at a time and compact the live
// ones in ascending order.
__global__ __launch_bounds__(256) void mask_lists_kernel(const MaskArgs a) {
  const MaskLayout& ml = a.ml;
  const int lane = threadIdx.x & 63;
  const int64_t np = (int64_t)ml.Bm * ml.Hm;
  int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int Tq = a.Tq;
  const bool causal = a.is_causal != 0;
  int kind;
  if (gw < np * ml.nfq) kind = 0;
  else if ((gw -= np * ml.nfq) < np * ml.nkb) kind = 1;
  else if ((gw -= np * ml.nkb) < np * ml.ndq) kind = 2;
  else return;
  const int per = kind == 0 ? ml.nfq : (kind == 1 ? ml.nkb : ml.ndq);
  const int pm = (int)(gw / per), unit = (int)(gw - (int64_t)pm * per);
  const uint8_t* blk = (const uint8_t*)(a.ws + ml.blk + pm * ml.pblk);
  int32_t* lst;
  int ncand;
  if (kind == 0) {
    lst = (int32_t*)(a.ws + ml.lfwd + pm * ml.plfwd) + (int64_t)unit * (1 + ml.nft);
    ncand = ml.nft;
  } else if (kind == 1) {
    lst = (int32_t*)(a.ws + ml.lkv + pm * ml.plkv) + (int64_t)unit * (1 + ml.nq32);
    ncand = ml.nq32;
  } else {
    lst = (int32_t*)(a.ws + ml.ldq + pm * ml.pldq) + (int64_t)unit * (1 + ml.nk32);
    ncand = ml.nk32;
  }
  int count = 0;
  for (int base = 0; base < ncand; base += 64) {
    const int cand = base + lane;
    bool live = false, full = true;
    if (cand < ncand) {
      // every block state is loaded before any is tested (predicated loads,
      // issued together: the scan is latency-bound otherwise)
      if (kind == 0) {
        // 256 rows x 64 keys: row blocks 8 unit .. +7, key blocks 2 cand, +1
        const int q_last = min(Tq - 1, kFwdRows * unit + kFwdRows - 1);
        if (!causal || kFwdKeys * cand <= q_last) {
          uint8_t st[8][2];
#pragma unroll
          for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              const int rb = 8 * unit + r, kb = 2 * cand + c;
              st[r][c] = (rb < ml.nq32 && kb < ml.nk32) ? blk[(int64_t)rb * ml.nk32 + kb] : 2;
            }
#pragma unroll
          for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              const int rb = 8 * unit + r, kb = 2 * cand + c;
              if (rb < ml.nq32 && kb < ml.nk32) live |= st[r][c] != 0;
              full &= st[r][c] == 2;
            }
        }
      } else if (kind == 1) {
        // 128 keys x 32 rows: key blocks 4 unit .. +3, row block cand
        if (!causal || min(Tq - 1, 32 * cand + 31) >= kKv2Keys * unit) {
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int kb = 4 * unit + c;
            if (kb < ml.nk32) live |= blk[(int64_t)cand * ml.nk32 + kb] != 0;
          }
        }
      } else {
        // 256 rows x 32 keys: row blocks 8 unit .. +7, key block cand
        const int q_last = min(Tq - 1, kDqDsRows * unit + kDqDsRows - 1);
        if (!causal || 32 * cand <= q_last) {
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            const int rb = 8 * unit + r;
            if (rb < ml.nq32) live |= blk[(int64_t)rb * ml.nk32 + cand] != 0;
          }
        }
      }
    }
    const uint64_t bal = __builtin_amdgcn_ballot_w64(live);
    const int pos = count + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
    if (live) lst[1 + pos] = (kind == 0 && full) ? (int32_t)(0x80000000u | (uint32_t)cand) : cand;
    count += __builtin_popcountll(bal);
  }
  if (lane == 0) lst[0] = count;
}

// One workgroup per (plane, list kind): the units of the lists in count
// order, largest first, ties by unit, by a counting sort over the counts
// (0 .. m, m the largest possible count: the tiles, steps or key steps of a
// list row):
//   1. histogram of the counts (atomic adds);
//   2. bin offsets, descending: start(c) = #units with a count above c (each
//      thread sums a contiguous range of bins, a log-step scan over the 256
//      partial sums, then each thread writes its range's offsets);
//   3. stable scatter: units in chunks of 256, in unit order; a unit's rank
//      among the units of its chunk with the same count (the chunk's counts
//      in LDS) added to its bin's offset, which the chunk's last such unit
//      then advances.
// O(n + m) work (an all-pairs ranking is O(n^2) in one workgroup).  The
// histogram sits in LDS when it fits (m < kHistLds), else in the workspace
// (hist), read and written with device-scope atomics (the L2: no wave reads
// a stale line from its CU's L1) between device-scope fences.
constexpr int kHistLds = 4096;

struct LdsHist {
  int32_t* h;
  __device__ int32_t ld(int c) const { return h[c]; }
  __device__ void st(int c, int32_t v) const { h[c] = v; }
  __device__ void add1(int c) const { atomicAdd(h + c, 1); }
  __device__ void sync() const { __syncthreads(); }
};
struct GlobalHist {
  int32_t* h;
  __device__ int32_t ld(int c) const { return __hip_atomic_load(h + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
  __device__ void st(int c, int32_t v) const { __hip_atomic_store(h + c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
  __device__ void add1(int c) const { __hip_atomic_fetch_add(h + c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
  __device__ void sync() const {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
};

template <typename Hist>
__device__ void order_units(const Hist& H, const int32_t* cnt, int64_t stride, int n, int m, int32_t* ord,
                            int32_t* part, int32_t* cs) {
  const int tid = threadIdx.x;
  // 1. histogram
  for (int c = tid; c <= m; c += 256) H.st(c, 0);
  H.sync();
  for (int i = tid; i < n; i += 256) H.add1(cnt[i * stride]);
  H.sync();
  // 2. descending offsets: thread t owns bins [lo, hi); the bins of the
  // threads above it come first in the order
  const int per = (m + 1 + 255) / 256;
  const int lo = min(m + 1, tid * per), hi = min(m + 1, lo + per);
  int32_t sum = 0;
  for (int c = lo; c < hi; ++c) sum += H.ld(c);
  part[tid] = sum;
  __syncthreads();
  // inclusive suffix sums over the 256 partial sums, log steps
  for (int d = 1; d < 256; d <<= 1) {
    const int32_t x = tid + d < 256 ? part[tid + d] : 0;
    __syncthreads();
    part[tid] += x;
    __syncthreads();
  }
  int32_t above = part[tid] - sum;   // units in the bins of the threads above
  for (int c = hi - 1; c >= lo; --c) {
    const int32_t h = H.ld(c);
    H.st(c, above);
    above += h;
  }
  H.sync();
  // 3. stable scatter
  for (int i0 = 0; i0 < n; i0 += 256) {
    const int i = i0 + tid, nc = min(256, n - i0);
    const int c = i < n ? cnt[i * stride] : -1;
    cs[tid] = c;
    __syncthreads();
    int r = 0;
    bool last = true;
    for (int j = 0; j < nc; ++j) {
      const bool same = cs[j] == c;
      r += (same & (j < tid)) ? 1 : 0;
      last &= !(same & (j > tid));
    }
    const int32_t base = i < n ? H.ld(c) : 0;
    if (i < n) ord[base + r] = i;
    __syncthreads();   // every offset of this chunk read before any advances
    if (i < n && last) H.st(c, base + r + 1);
    H.sync();
  }
}

__global__ __launch_bounds__(256) void mask_order_kernel(const MaskArgs a) {
  const MaskLayout& ml = a.ml;
  const int pm = blockIdx.x, kind = blockIdx.y;
  const int n = kind == 0 ? ml.nfq : (kind == 1 ? ml.nkb : ml.ndq);
  const int m = kind == 0 ? ml.nft : (kind == 1 ? ml.nq32 : ml.nk32);   // largest possible count
  const int32_t* cnt = (const int32_t*)(a.ws + (kind == 0 ? ml.lfwd + pm * ml.plfwd
                                                : (kind == 1 ? ml.lkv + pm * ml.plkv : ml.ldq + pm * ml.pldq)));
  int32_t* ord = (int32_t*)mask_order(ml, a.ws, pm, kind);
  __shared__ int32_t part[256], cs[256], hl[kHistLds];
  if (m < kHistLds) {
    order_units(LdsHist{hl}, cnt, 1 + m, n, m, ord, part, cs);
  } else {
    int32_t* hg = (int32_t*)(a.ws + ml.hist + pm * ml.phist) +
                  (kind == 0 ? 0 : (kind == 1 ? ml.nft + 1 : ml.nft + 1 + ml.nq32 + 1));
    order_units(GlobalHist{hg}, cnt, 1 + m, n, m, ord, part, cs);
  }
}

}  // namespace

hipError_t launch_mask_prepare(const MaskArgs& a, hipStream_t s) {
  const MaskLayout& ml = a.ml;
  const dim3 g1((unsigned)((a.Tk + kKeys - 1) / kKeys), (unsigned)min((a.Tq + kRows - 1) / kRows, 65535),
                (unsigned)min(ml.Bm * ml.Hm, 65535));
  hipLaunchKernelGGL(mask_bits_kernel, g1, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t nl = (int64_t)ml.Bm * ml.Hm * (ml.nfq + ml.nkb + ml.ndq);
  hipLaunchKernelGGL(mask_lists_kernel, dim3((unsigned)((nl + 3) / 4)), dim3(256), 0, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(mask_order_kernel, dim3((unsigned)(ml.Bm * ml.Hm), 3), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace fa
