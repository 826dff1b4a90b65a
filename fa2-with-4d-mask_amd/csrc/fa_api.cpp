// C ABI of libfa2_4d_mask.so: argument validation, planning, kernel launch.
//
// Every entry point checks its arguments on the host before any HIP call and
// returns an FA_ERR_* code with nothing enqueued when they are unusable, so the
// validation paths run (and are tested) on machines without a GPU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "fa2_4d_mask.h"
#include "fa_kernels.h"

namespace fa {
int fwd_block_rows();
int dq_block_rows();
// fa_noalloc.hip: the allocation-free backward's device scratch
int64_t noalloc_scratch_bytes();
hipError_t scratch_device_ptr(void** out);
hipError_t launch_fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t s);
}  // namespace fa

namespace {

thread_local char g_err[512] = "no error";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Rows of a [.., T, H, D] operand must start on 16 bytes: base aligned and the
// batch/time/head strides multiples of 8 elements (16-bit data).
int check_operand(const char* name, const void* p, int64_t sb, int64_t st, int64_t sh) {
  if (!p) return fail(FA_ERR_NULL, "%s is NULL", name);
  if (!aligned16(p)) return fail(FA_ERR_STRIDE, "%s base pointer is not 16-byte aligned", name);
  if (sb % 8 || st % 8 || sh % 8)
    return fail(FA_ERR_STRIDE, "%s strides (b=%lld, t=%lld, h=%lld) must be multiples of 8 elements", name,
                (long long)sb, (long long)st, (long long)sh);
  return FA_OK;
}

// Rows of every head below 2^31 - 2^16: 32-bit row indices with room to
// round any count up to a whole tile.
constexpr int64_t kMaxRows = (1LL << 31) - (1LL << 16);
// Products of non-negative sizes in the plans saturate at kSizeSat, so that
// shapes whose dS tiles no device could hold still plan (to the recompute
// route) with defined arithmetic; kSizeSat leaves room for doubling and sums.
constexpr int64_t kSizeSat = INT64_MAX / 8;
int64_t sat_mul(int64_t a, int64_t b) {
  if (a == 0 || b == 0) return 0;
  return a > kSizeSat / b ? kSizeSat : std::min(a * b, kSizeSat);
}

int check_dims(int32_t B, int32_t Tq, int32_t Tk, int32_t Hq, int32_t Hk, int32_t D, int32_t dtype, float scale) {
  if (B < 1 || Tq < 1 || Tk < 1 || Hq < 1 || Hk < 1)
    return fail(FA_ERR_SHAPE, "sizes must be >= 1 (B=%d Tq=%d Tk=%d Hq=%d Hk=%d)", B, Tq, Tk, Hq, Hk);
  if (Hq % Hk != 0)
    return fail(FA_ERR_SHAPE, "query heads (%d) must be divisible by key/value heads (%d)", Hq, Hk);
  if (D != 64 && D != 128 && D != 256) return fail(FA_ERR_HEAD_DIM, "head_dim %d not supported (64, 128, 256)", D);
  if (dtype != FA_DTYPE_BF16 && dtype != FA_DTYPE_FP16) return fail(FA_ERR_DTYPE, "unsupported dtype code %d", dtype);
  if (!std::isfinite(scale)) return fail(FA_ERR_SCALE, "scale must be finite");
  // 32-bit indices inside the kernels and the host: rows of every head must
  // fit, with room to round any of them up to a whole tile.
  if ((int64_t)B * Hq * (int64_t)Tq >= kMaxRows || (int64_t)B * Hk * (int64_t)Tk >= kMaxRows)
    return fail(FA_ERR_SHAPE, "problem too large for 32-bit row indices (B*H*T must stay below 2^31 - 2^16)");
  return FA_OK;
}

int check_mask_score(const uint8_t* mask, int64_t msb, int64_t msh, int64_t msq, const float* score, int64_t ssb,
                     int64_t ssh, int64_t ssq) {
  if (mask && (msb < 0 || msh < 0 || msq < 0)) return fail(FA_ERR_STRIDE, "mask strides must be non-negative");
  if (score && (ssb < 0 || ssh < 0 || ssq < 0)) return fail(FA_ERR_STRIDE, "score strides must be non-negative");
  return FA_OK;
}

fa::MaskLayout layout_of(int32_t B, int32_t Hq, int32_t Tq, int32_t Tk, int64_t msb, int64_t msh) {
  return fa::mask_layout(B, Hq, Tq, Tk, msb == 0, msh == 0);
}

// A prepared mask is required beside a mask; it must be 256-byte aligned.
int check_mask_ws(const uint8_t* mask, const void* ws) {
  if (!mask) return FA_OK;
  if (!ws) return fail(FA_ERR_WORKSPACE, "a mask needs its prepared workspace (fa_mask_prepare): mask_ws is NULL");
  if ((uintptr_t)ws % 256) return fail(FA_ERR_STRIDE, "mask_ws must be 256-byte aligned");
  return FA_OK;
}

int launch_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(FA_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return FA_OK;
}

// dS tiles (16-bit, every stored 32x32 block; causal: blocks on or below the
// diagonal) handed from the dK/dV kernel to the dQ kernel.  The workspace
// holds the planes of a slice of (batch, kv-head) units, as many as fit the
// caller's limit (all of them when they fit), in as few slices of nearly
// equal size as that allows: the backward then runs the two kernels once per
// slice.  0 units: not even one unit fits.
// With a mask or a score each tile is a pair: dS rounded, then its rounding
// residual (the dQ kernel adds both products).
int ds_tile_parts(const FaBwdParams* p) { return p->mask || p->score ? 2 : 1; }
// Default limit (ds_limit_bytes = 0): a constant, so the route, the slices and
// the head-group split depend on the problem alone.  The headline shape (B1
// T8192 Hq32 Hk8 D128) needs exactly 4 GiB non-causal and runs unsliced.
constexpr int64_t kDsLimitDefault = (int64_t)4 << 30;
int64_t ds_unit_elems(const FaBwdParams* p) {
  const int64_t nq32 = (p->seqlen_q + 31) / 32, nk32 = (p->seqlen_k + 31) / 32;
  const int64_t plane = fa::ds_row(nq32, nk32, p->is_causal != 0);
  // one unit: the group's planes
  return sat_mul(sat_mul(sat_mul(p->heads_q / p->heads_k, plane), 1024), ds_tile_parts(p));
}
// The caller's limit, below kSizeSat / 4 (beyond any device): saturated sizes
// then never fit it.
int64_t ds_limit_of(const FaBwdParams* p) {
  return p->ds_limit_bytes == 0 ? kDsLimitDefault : std::min<int64_t>(p->ds_limit_bytes, kSizeSat / 4);
}

// Row ranges.  Without a mask the dS route can run over ranges of query rows
// instead of groups of units: each range's dK/dV launch covers every unit
// (the workgroups of the whole problem, each over the range's rows) and adds
// its partial dK/dV to fp32 sums; its dQ launch completes dQ for the range's
// rows.  Ranges start on 512-row boundaries (whole dQ row blocks); their
// count is the smallest the limit allows, their tile counts balanced.  Used
// when the tiles exceed the limit and either not even one unit fits it, or
// the problem is causal (unit slices of a causal problem split each head
// group to balance their workgroups, through fp32 slabs: measured 5-25 %
// slower than ranges at 0.5-4 GiB; non-causal unit slices ran 1-3 % faster
// than ranges).  With a mask the per-key-block lists of live steps are not
// ranged: below one unit such problems recompute dQ.
constexpr int kRangeSteps = 16;
// bytes of the dS tiles of query steps [lo, hi) over every (batch, head)
int64_t range_bytes(const FaBwdParams* p, int lo, int hi) {
  const int64_t nk32 = (p->seqlen_k + 31) / 32;
  const bool causal = p->is_causal != 0;
  const int64_t steps = fa::ds_row(hi, nk32, causal) - fa::ds_row(lo, nk32, causal);
  return sat_mul(sat_mul(sat_mul(sat_mul((int64_t)p->batch * p->heads_q, steps), 1024), ds_tile_parts(p)), 2);
}
// Greedy ranges of at most `cap` bytes: their count (-1 if one 512-row
// chunk exceeds it); step bounds into `bounds` when given.
int ranges_under(const FaBwdParams* p, int64_t cap, std::vector<int>* bounds) {
  const int nq32 = (p->seqlen_q + 31) / 32;
  if (bounds) bounds->assign(1, 0);
  int n = 0;
  for (int lo = 0; lo < nq32;) {
    int hi = lo;
    while (hi < nq32 && range_bytes(p, lo, std::min(hi + kRangeSteps, nq32)) <= cap) hi = std::min(hi + kRangeSteps, nq32);
    if (hi == lo) return -1;
    ++n;
    if (bounds) bounds->push_back(hi);
    lo = hi;
  }
  return n;
}
// Number of row ranges (0: none), step bounds into `bounds` (n + 1 entries).
int row_ranges(const FaBwdParams* p, std::vector<int>* bounds) {
  if (p->mask || p->head_dim > 128) return 0;
  const int64_t limit = ds_limit_of(p);
  const int64_t unit = ds_unit_elems(p);
  if (limit < 0 || unit <= 0) return 0;
  const int64_t total = range_bytes(p, 0, (p->seqlen_q + 31) / 32);
  if (total <= limit) return 0;                                           // one launch
  if (!p->is_causal && limit / (2 * unit) >= 1) return 0;                 // unit slices
  const int n = ranges_under(p, limit, nullptr);
  if (n < 2) return 0;   // a 512-row chunk of every unit exceeds the limit: dQ is recomputed
  // the smallest cap that keeps n ranges balances their tile counts
  int64_t lo = (total + n - 1) / n - 1, hi = limit;   // count(lo) > n (or -1), count(hi) == n
  while (hi - lo > 1) {
    const int64_t mid = lo + (hi - lo) / 2;
    const int c = ranges_under(p, mid, nullptr);
    if (c > 0 && c <= n) hi = mid;
    else lo = mid;
  }
  return ranges_under(p, hi, bounds);
}

// Parts of a head group.  With a mask (whose lists of live steps are not
// ranged), when not even one unit's tiles fit the limit, the head group
// splits into parts of whole query heads -- the dK/dV kernel's head-group
// split, one fp32 slab per part summed by fa_bwd_finalize -- and each slice
// holds the planes of some parts of one unit, in nearly equal slices.  One
// head per part (unless the caller sets the split): a slice's planes then
// give the most workgroups (two-head parts halve them for the same planes:
// T 20000 with packed documents, fwd+bwd 3.7 ms against 3.3 with one-head
// parts).  Returns the split (0: none) and the parts per slice.
int part_split(const FaBwdParams* p, int* per) {
  if (!p->mask || p->head_dim > 128) return 0;
  const int64_t limit = ds_limit_of(p), unit = ds_unit_elems(p);
  if (limit < 0 || unit <= 0 || limit / (2 * unit) >= 1) return 0;
  const int G = p->heads_q / p->heads_k;
  const int s = p->kv_split > 0 ? p->kv_split : G;
  if (s < 2 || G % s != 0) return 0;
  const int64_t part = 2 * (unit / s);   // bytes of one part's planes
  if (part > limit) return 0;
  if (per) {
    const int nsl = (int)((s + limit / part - 1) / (limit / part));   // slices per unit
    *per = (s + nsl - 1) / nsl;
  }
  return s;
}

int64_t ds_slice_units(const FaBwdParams* p) {
  if (p->head_dim > 128) return 0;   // head dim 256: dQ is always recomputed
  const int64_t limit = ds_limit_of(p);
  if (limit < 0) return 0;
  const int64_t units = (int64_t)p->batch * p->heads_k, unit = ds_unit_elems(p);
  if (unit <= 0) return units;
  if (row_ranges(p, nullptr) > 0) return units;   // row ranges hold every unit
  const int64_t most = std::min(units, limit / (2 * unit));
  if (most <= 0) return 0;
  // as few slices as the limit allows, of (nearly) equal size
  const int64_t slices = (units + most - 1) / most;
  return (units + slices - 1) / slices;
}
int64_t ds_elems(const FaBwdParams* p) {
  int per = 0;
  if (const int s = part_split(p, &per)) return per * (ds_unit_elems(p) / s);
  std::vector<int> rb;
  const int nr = row_ranges(p, &rb);
  if (nr > 0) {
    int64_t most = 0;
    for (int r = 0; r < nr; ++r) most = std::max(most, range_bytes(p, rb[r], rb[r + 1]) / 2);
    return most;
  }
  return ds_slice_units(p) * ds_unit_elems(p);
}
// launches of the dS route: unit slices, or row ranges
int ds_slices(const FaBwdParams* p) {
  const int nr = row_ranges(p, nullptr);
  if (nr > 0) return nr;
  int parts = 0;
  if (const int s = part_split(p, &parts)) return p->batch * p->heads_k * ((s + parts - 1) / parts);
  const int64_t per = ds_slice_units(p);
  return per > 0 ? (int)(((int64_t)p->batch * p->heads_k + per - 1) / per) : 0;
}

// How the backward runs.  With the dS tiles: the pipelined dK/dV kernel
// stores dS and a dQ kernel streams it, writing dQ (deterministic) or adding
// fp32 partials over key ranges atomically (atomic, below one row block per
// CU).  Without them, in both modes: the dK/dV kernel alone, then a dQ kernel
// that recomputes S, P and dP -- deterministic, no atomics, and faster than
// adding dQ with fp32 atomics from the dK/dV kernel as the reference's atomic
// kernel does (measured with such a fused kernel: H 7.7 against 4.8 ms
// fwd+bwd, causal 5.1 against 2.7, config M 2.0 against 1.5).
// Head dim 256 always takes the recompute route (its dK/dV kernels store no
// dS tiles and add no atomics).
enum Route { kDsAtomic, kDsDet, kRecomputeDet };
Route route_of(const FaBwdParams* p) {
  if (p->head_dim > 128) return kRecomputeDet;
  const bool ds = ds_elems(p) > 0;
  if (!ds) return kRecomputeDet;
  return p->atomic_dq ? kDsAtomic : kDsDet;
}

// Key ranges of the atomic dQ-from-dS kernel: at least 2, more while the grid
// is below ~1024 workgroups and each range keeps >= 4 key steps.
// Workgroups of one dQ-from-dS launch (one slice of units) at `rows` query
// rows each, and the CU count they are measured against.
int64_t dq_groups(const FaBwdParams* p, int rows) {
  return ds_slice_units(p) * (p->heads_q / p->heads_k) * ((p->seqlen_q + rows - 1) / rows);
}
constexpr int64_t kCus = 256;

// Atomic mode with the dS tiles: when the 256-row blocks alone give every CU
// a workgroup, each workgroup owns its rows and writes dQ (split 1: no fp32
// atomics, no zeroing, no conversion -- 20-70 % faster than adding partials);
// below that, 2-8 key ranges per block are added with fp32 atomics, more
// while the grid is below ~1024 workgroups and each range keeps >= 4 steps.
int dq_split_of(const FaBwdParams* p) {
  // (row ranges and head-group parts: dQ written per launch)
  if (route_of(p) != kDsAtomic || row_ranges(p, nullptr) > 0 || part_split(p, nullptr) > 0) return 1;
  const int64_t nblk = dq_groups(p, fa::kDqDsRows);
  const int nks = (p->seqlen_k + 31) / 32;
  if (nblk >= kCus || nks < 2) return 1;
  int split = 2;
  while (split < 8 && nblk * split < 1024 && nks / (2 * split) >= 4) split *= 2;
  return split;
}

// keys per workgroup of the dK/dV launch(es) of the route
int kv_block_keys(const FaBwdParams* p) {
  if (p->head_dim > 128) return fa::kv_wide_block_keys();
  return fa::dkdv2_block_keys();
}

// dQ accumulated with fp32 atomics into dq_accum (then converted)
bool dq_atomics(const FaBwdParams* p) {
  const Route r = route_of(p);
  return r == kDsAtomic && dq_split_of(p) > 1;
}

// query rows per workgroup of the dQ-from-dS kernel: 512 (8 waves sharing
// each K tile) when dQ is written directly at head dim 128 without a mask or
// a score (whose tile pairs double the staging) and that still gives every CU
// a workgroup, else 256
int dq_rows(const FaBwdParams* p) {
  if (p->head_dim != 128 || p->mask || p->score || dq_atomics(p)) return fa::kDqDsRows;
  return dq_groups(p, fa::kDqDsRowsWide) >= kCus ? fa::kDqDsRowsWide : fa::kDqDsRows;
}

int choose_split(const FaBwdParams* p) {
  if (p->kv_split > 0) return p->kv_split;
  if (const int s = part_split(p, nullptr)) return s;
  const bool ranged = row_ranges(p, nullptr) > 0;
  if (ranged && !p->is_causal) return 1;   // every unit in each launch, equal work: one fp32 sum
  const int G = p->heads_q / p->heads_k;
  const int kb = kv_block_keys(p);
  const int nkt = (p->seqlen_k + kb - 1) / kb;
  const Route r = route_of(p);
  const int64_t units = r == kDsAtomic || r == kDsDet ? ds_slice_units(p) : (int64_t)p->batch * p->heads_k;
  const int64_t base = units * nkt;   // workgroups of one launch without a split
  // two workgroups per CU on a 256-CU part.  Causal workgroups differ in work
  // (key block kt walks the rows from kt on); when the backward runs in slices
  // (long sequences) twice as many keep each slice's tail short (measured:
  // T 16384 causal 10.1 -> 8.9 ms), while a single launch at the headline
  // size is faster without the split's fp32 slabs.  Sliced non-causal
  // launches aim at one workgroup per CU (equal work: one round), which
  // halves the split and its slabs (H with a 1 GiB limit: -2.4 %).
  // Causal row ranges: the first range's work per key block is a triangle
  // (its longest workgroup walks several times the average), which a split
  // of the head group evens out; each part keeps its own fp32 slab across
  // the ranges.
  const bool sliced = ranged || units < (int64_t)p->batch * p->heads_k;
  const int64_t target = sliced ? (p->is_causal ? 1024 : kCus) : 512;
  int split = 1;
  while (split * 2 <= G && G % (split * 2) == 0 && base * split < target) split *= 2;
  return split;
}

// The delta workspace holds Delta [B, Hq, Tq], then the LSE the backward
// kernels read (written by the preprocess).
float* lse_b_of(const FaBwdParams* p) {
  return p->delta + (int64_t)p->batch * p->heads_q * p->seqlen_q;
}

void fill_scales(float scale, float* scale_log2_fwd, float* qsign, int* zero, float* scale_log2_bwd) {
  *zero = scale == 0.f;
  *qsign = scale < 0.f ? -1.f : 1.f;
  const float l2e = 1.4426950408889634f;
  *scale_log2_fwd = *zero ? 1.f : std::fabs(scale) * l2e;
  *scale_log2_bwd = *zero ? 1.f : scale * l2e;
}

}  // namespace

extern "C" {

int fa_abi_version(void) { return FA_ABI_VERSION; }

static int check_mask_params(const FaMaskParams* p) {
  if (!p) return fail(FA_ERR_NULL, "params is NULL");
  if (p->batch < 1 || p->seqlen_q < 1 || p->seqlen_k < 1 || p->heads_q < 1)
    return fail(FA_ERR_SHAPE, "sizes must be >= 1 (B=%d Tq=%d Tk=%d Hq=%d)", p->batch, p->seqlen_q, p->seqlen_k,
                p->heads_q);
  if (!p->mask) return fail(FA_ERR_NULL, "mask is NULL");
  if (p->mask_stride_b < 0 || p->mask_stride_h < 0 || p->mask_stride_q < 0)
    return fail(FA_ERR_STRIDE, "mask strides must be non-negative");
  const fa::MaskLayout ml = layout_of(p->batch, p->heads_q, p->seqlen_q, p->seqlen_k, p->mask_stride_b,
                                      p->mask_stride_h);
  if ((int64_t)ml.Bm * ml.Hm >= (1LL << 31))
    return fail(FA_ERR_SHAPE, "mask has too many planes (%d x %d) for 32-bit plane indices", ml.Bm, ml.Hm);
  return FA_OK;
}

int fa_mask_plan(const FaMaskParams* p, int64_t* workspace_bytes) {
  int st = check_mask_params(p);
  if (st) return st;
  if (!workspace_bytes) return fail(FA_ERR_NULL, "workspace_bytes is NULL");
  *workspace_bytes = layout_of(p->batch, p->heads_q, p->seqlen_q, p->seqlen_k, p->mask_stride_b, p->mask_stride_h).total;
  return FA_OK;
}

int fa_mask_prepare(const FaMaskParams* p) {
  int st = check_mask_params(p);
  if (st) return st;
  if (!p->workspace) return fail(FA_ERR_WORKSPACE, "workspace is NULL");
  if ((uintptr_t)p->workspace % 256) return fail(FA_ERR_STRIDE, "workspace must be 256-byte aligned");
  fa::MaskArgs a{};
  a.mask = p->mask;
  a.msb = p->mask_stride_b; a.msh = p->mask_stride_h; a.msq = p->mask_stride_q;
  a.Tq = p->seqlen_q; a.Tk = p->seqlen_k;
  a.is_causal = p->is_causal != 0;
  a.vec16 = ((uintptr_t)p->mask % 16 == 0) && p->mask_stride_b % 16 == 0 && p->mask_stride_h % 16 == 0 &&
            p->mask_stride_q % 16 == 0;
  a.ws = (char*)p->workspace;
  a.ml = layout_of(p->batch, p->heads_q, p->seqlen_q, p->seqlen_k, p->mask_stride_b, p->mask_stride_h);
  return launch_status(fa::launch_mask_prepare(a, (hipStream_t)p->stream), "fa_mask_prepare");
}

const char* fa_last_error(void) { return g_err; }

int fa_fwd(const FaFwdParams* p) {
  if (!p) return fail(FA_ERR_NULL, "params is NULL");
  int st = check_dims(p->batch, p->seqlen_q, p->seqlen_k, p->heads_q, p->heads_k, p->head_dim, p->dtype, p->scale);
  if (st) return st;
  if ((st = check_operand("q", p->q, p->q_stride_b, p->q_stride_t, p->q_stride_h))) return st;
  if ((st = check_operand("k", p->k, p->k_stride_b, p->k_stride_t, p->k_stride_h))) return st;
  if ((st = check_operand("v", p->v, p->v_stride_b, p->v_stride_t, p->v_stride_h))) return st;
  if ((st = check_operand("o", p->o, p->o_stride_b, p->o_stride_t, p->o_stride_h))) return st;
  if (p->o_lo && (st = check_operand("o_lo", p->o_lo, p->o_lo_stride_b, p->o_lo_stride_t, p->o_lo_stride_h)))
    return st;
  if (!p->lse) return fail(FA_ERR_NULL, "lse is NULL");
  if ((st = check_mask_score(p->mask, p->mask_stride_b, p->mask_stride_h, p->mask_stride_q, p->score,
                             p->score_stride_b, p->score_stride_h, p->score_stride_q)))
    return st;
  if ((st = check_mask_ws(p->mask, p->mask_ws))) return st;

  // The forward stages K/V tiles with 32-bit buffer offsets (64 rows of a tile).
  if (p->k_stride_t < 0 || p->k_stride_t >= (1LL << 24) || p->v_stride_t < 0 || p->v_stride_t >= (1LL << 24))
    return fail(FA_ERR_STRIDE, "k/v time strides (%lld, %lld) must lie in [0, 2^24) elements",
                (long long)p->k_stride_t, (long long)p->v_stride_t);
  // ... and a wave's 32 score rows through one buffer with 32-bit offsets.
  if (p->score && (31 * p->score_stride_q + (int64_t)p->seqlen_k + 64) * 4 >= (1LL << 32))
    return fail(FA_ERR_STRIDE, "score query stride %lld: 32 score rows must span less than 4 GiB",
                (long long)p->score_stride_q);

  fa::FwdArgs a{};
  a.q = p->q; a.k = p->k; a.v = p->v; a.o = p->o; a.lse = p->lse;
  a.mask = p->mask; a.score = p->score;
  a.qsb = p->q_stride_b; a.qst = p->q_stride_t; a.qsh = p->q_stride_h;
  a.ksb = p->k_stride_b; a.kst = p->k_stride_t; a.ksh = p->k_stride_h;
  a.vsb = p->v_stride_b; a.vst = p->v_stride_t; a.vsh = p->v_stride_h;
  a.osb = p->o_stride_b; a.ost = p->o_stride_t; a.osh = p->o_stride_h;
  a.msb = p->mask_stride_b; a.msh = p->mask_stride_h; a.msq = p->mask_stride_q;
  a.ssb = p->score_stride_b; a.ssh = p->score_stride_h; a.ssq = p->score_stride_q;
  a.B = p->batch; a.Tq = p->seqlen_q; a.Tk = p->seqlen_k; a.Hq = p->heads_q; a.Hk = p->heads_k;
  a.G = p->heads_q / p->heads_k;
  const int fwd_rows = p->head_dim > 128 ? fa::fwd_wide_block_rows() : fa::fwd_block_rows();
  a.nqt = (p->seqlen_q + fwd_rows - 1) / fwd_rows;
  float sl2b;
  fill_scales(p->scale, &a.scale_log2, &a.qsign, &a.zero_scale, &sl2b);
  if (p->mask) {
    a.mws = (const char*)p->mask_ws;
    a.ml = layout_of(p->batch, p->heads_q, p->seqlen_q, p->seqlen_k, p->mask_stride_b, p->mask_stride_h);
  }
  if (p->o_lo && (p->mask || p->score)) {
    a.olo = p->o_lo;
    a.olsb = p->o_lo_stride_b; a.olst = p->o_lo_stride_t; a.olsh = p->o_lo_stride_h;
  }
  const hipStream_t s = (hipStream_t)p->stream;
  if (p->head_dim > 128) return launch_status(fa::launch_fwd_wide(a, p->dtype, p->is_causal != 0, s), "fa_fwd");
  return launch_status(fa::launch_fwd(a, p->head_dim, p->dtype, p->is_causal != 0, s), "fa_fwd");
}

static int check_bwd(const FaBwdParams* p, int split) {
  int st = check_dims(p->batch, p->seqlen_q, p->seqlen_k, p->heads_q, p->heads_k, p->head_dim, p->dtype, p->scale);
  if (st) return st;
  if ((st = check_operand("q", p->q, p->q_stride_b, p->q_stride_t, p->q_stride_h))) return st;
  if ((st = check_operand("k", p->k, p->k_stride_b, p->k_stride_t, p->k_stride_h))) return st;
  if ((st = check_operand("v", p->v, p->v_stride_b, p->v_stride_t, p->v_stride_h))) return st;
  if ((st = check_operand("o", p->o, p->o_stride_b, p->o_stride_t, p->o_stride_h))) return st;
  if ((st = check_operand("dout", p->dout, p->do_stride_b, p->do_stride_t, p->do_stride_h))) return st;
  if ((st = check_operand("dq", p->dq, p->dq_stride_b, p->dq_stride_t, p->dq_stride_h))) return st;
  if ((st = check_operand("dk", p->dk, p->dk_stride_b, p->dk_stride_t, p->dk_stride_h))) return st;
  if ((st = check_operand("dv", p->dv, p->dv_stride_b, p->dv_stride_t, p->dv_stride_h))) return st;
  if (p->o_lo && (st = check_operand("o_lo", p->o_lo, p->o_lo_stride_b, p->o_lo_stride_t, p->o_lo_stride_h)))
    return st;
  // The dK/dV kernel stages Q/dO tiles with 32-bit buffer offsets (32 rows of a tile).
  // The dQ kernel stages K tiles the same way.
  if (p->q_stride_t < 0 || p->q_stride_t >= (1LL << 24) || p->do_stride_t < 0 || p->do_stride_t >= (1LL << 24) ||
      p->k_stride_t < 0 || p->k_stride_t >= (1LL << 24))
    return fail(FA_ERR_STRIDE, "q/dout/k time strides (%lld, %lld, %lld) must lie in [0, 2^24) elements",
                (long long)p->q_stride_t, (long long)p->do_stride_t, (long long)p->k_stride_t);
  // ... and reaches a tile's first row of Q / dO with a 32-bit scalar byte offset.
  const int64_t qspan = (int64_t)(p->seqlen_q + 32) * 2 * (p->q_stride_t > p->do_stride_t ? p->q_stride_t : p->do_stride_t);
  if (qspan >= (1LL << 32))
    return fail(FA_ERR_STRIDE, "seqlen_q * q/dout time stride too large (%lld bytes, the limit is 2^32)", (long long)qspan);
  // The dK/dV kernel reads a step's 32 score rows through one buffer with
  // 32-bit offsets, as the forward does a wave's.
  if (p->score && (31 * p->score_stride_q + (int64_t)p->seqlen_k + 64) * 4 >= (1LL << 32))
    return fail(FA_ERR_STRIDE, "score query stride %lld: 32 score rows must span less than 4 GiB",
                (long long)p->score_stride_q);
  if (!p->lse) return fail(FA_ERR_NULL, "lse is NULL");
  if (!p->delta) return fail(FA_ERR_NULL, "delta is NULL");
  if (!p->dead_flags) return fail(FA_ERR_NULL, "dead_flags is NULL");
  if (dq_atomics(p) && !p->dq_accum) return fail(FA_ERR_WORKSPACE, "atomic dQ needs dq_accum (plan.needs_dq_accum)");
  if (dq_atomics(p) && !aligned16(p->dq_accum)) return fail(FA_ERR_STRIDE, "dq_accum must be 16-byte aligned");
  const int G = p->heads_q / p->heads_k;
  if (split < 1 || G % split != 0) return fail(FA_ERR_SHAPE, "kv_split %d must divide the group size %d", split, G);
  if (split > 1 && (!p->dk_accum || !p->dv_accum))
    return fail(FA_ERR_WORKSPACE, "kv_split %d needs dk_accum and dv_accum", split);
  if (split > 1 && (!aligned16(p->dk_accum) || !aligned16(p->dv_accum)))
    return fail(FA_ERR_STRIDE, "dk_accum/dv_accum must be 16-byte aligned");
  if (row_ranges(p, nullptr) > 0) {
    if (!p->dk_accum || !p->dv_accum)
      return fail(FA_ERR_WORKSPACE, "the backward over row ranges needs dk_accum and dv_accum (plan.dkv_accum_elems)");
    if (!aligned16(p->dk_accum) || !aligned16(p->dv_accum))
      return fail(FA_ERR_STRIDE, "dk_accum/dv_accum must be 16-byte aligned");
  }
  if (ds_elems(p) > 0 && !p->ds_tiles) return fail(FA_ERR_WORKSPACE, "dQ from dS tiles needs ds_tiles (plan.ds_elems)");
  if (ds_elems(p) > 0 && p->ds_tiles_elems < ds_elems(p))
    return fail(FA_ERR_WORKSPACE, "ds_tiles holds %lld elements, the plan needs %lld (with a mask or a score each "
                "block is a pair of tiles: plan with mask/score set)", (long long)p->ds_tiles_elems,
                (long long)ds_elems(p));
  if (ds_elems(p) > 0 && !aligned16(p->ds_tiles)) return fail(FA_ERR_STRIDE, "ds_tiles must be 16-byte aligned");
  if ((st = check_mask_ws(p->mask, p->mask_ws))) return st;
  return check_mask_score(p->mask, p->mask_stride_b, p->mask_stride_h, p->mask_stride_q, p->score,
                          p->score_stride_b, p->score_stride_h, p->score_stride_q);
}

int fa_bwd_plan(const FaBwdParams* p, FaBwdPlan* plan) {
  if (!p || !plan) return fail(FA_ERR_NULL, "params or plan is NULL");
  int st = check_dims(p->batch, p->seqlen_q, p->seqlen_k, p->heads_q, p->heads_k, p->head_dim, p->dtype, p->scale);
  if (st) return st;
  const int split = choose_split(p);
  const int G = p->heads_q / p->heads_k;
  if (split < 1 || G % split != 0) return fail(FA_ERR_SHAPE, "kv_split %d must divide the group size %d", split, G);
  plan->kv_split = split;
  plan->needs_dq_accum = dq_atomics(p) ? 1 : 0;
  plan->dq_accum_elems = dq_atomics(p) ? (int64_t)p->batch * p->seqlen_q * p->heads_q * p->head_dim : 0;
  // one fp32 slab per head-group part, fully overwritten (nothing to zero)
  plan->dkv_accum_zeroed = 0;
  plan->dkv_accum_elems = split > 1 ? (int64_t)split * p->batch * p->seqlen_k * p->heads_k * p->head_dim : 0;
  // row ranges: one fp32 sum (split 1) or slab per split each for dK and dV,
  // written by the first range
  if (row_ranges(p, nullptr) > 0)
    plan->dkv_accum_elems = (int64_t)split * p->batch * p->seqlen_k * p->heads_k * p->head_dim;
  plan->ds_elems = ds_elems(p);
  plan->dq_split = dq_split_of(p);
  return FA_OK;
}

int fa_bwd_preprocess(const FaBwdParams* p) {
  if (!p) return fail(FA_ERR_NULL, "params is NULL");
  const int split = choose_split(p);
  int st = check_bwd(p, split);
  if (st) return st;
  fa::PreArgs a{};
  a.o = p->o; a.dout = p->dout; a.lse = p->lse; a.dead = p->dead_flags;
  a.delta = p->delta;
  a.lse_b = lse_b_of(p);
  a.dq_accum = dq_atomics(p) ? p->dq_accum : nullptr;
  a.osb = p->o_stride_b; a.ost = p->o_stride_t; a.osh = p->o_stride_h;
  a.dsb = p->do_stride_b; a.dst = p->do_stride_t; a.dsh = p->do_stride_h;
  a.olo = p->o_lo;
  a.olsb = p->o_lo_stride_b; a.olst = p->o_lo_stride_t; a.olsh = p->o_lo_stride_h;
  a.B = p->batch; a.Tq = p->seqlen_q; a.Hq = p->heads_q; a.Hk = p->heads_k; a.G = p->heads_q / p->heads_k;
  a.is_causal = p->is_causal != 0;
  if (p->mask) {
    a.mws = (const char*)p->mask_ws;
    a.ml = layout_of(p->batch, p->heads_q, p->seqlen_q, p->seqlen_k, p->mask_stride_b, p->mask_stride_h);
  }
  return launch_status(fa::launch_preprocess(a, p->head_dim, p->dtype, (hipStream_t)p->stream), "fa_bwd_preprocess");
}

static fa::BwdArgs bwd_args(const FaBwdParams* p, int split) {
  fa::BwdArgs a{};
  a.q = p->q; a.k = p->k; a.v = p->v; a.dout = p->dout;
  a.lse = lse_b_of(p); a.delta = p->delta; a.dead = p->dead_flags;
  a.mask = p->mask; a.score = p->score;
  a.dq_accum = p->dq_accum; a.dk_accum = p->dk_accum; a.dv_accum = p->dv_accum;
  a.dk = p->dk; a.dv = p->dv; a.dq = p->dq;
  a.qsb = p->q_stride_b; a.qst = p->q_stride_t; a.qsh = p->q_stride_h;
  a.ksb = p->k_stride_b; a.kst = p->k_stride_t; a.ksh = p->k_stride_h;
  a.vsb = p->v_stride_b; a.vst = p->v_stride_t; a.vsh = p->v_stride_h;
  a.dsb = p->do_stride_b; a.dst = p->do_stride_t; a.dsh = p->do_stride_h;
  a.dqsb = p->dq_stride_b; a.dqst = p->dq_stride_t; a.dqsh = p->dq_stride_h;
  a.dksb = p->dk_stride_b; a.dkst = p->dk_stride_t; a.dksh = p->dk_stride_h;
  a.dvsb = p->dv_stride_b; a.dvst = p->dv_stride_t; a.dvsh = p->dv_stride_h;
  a.msb = p->mask_stride_b; a.msh = p->mask_stride_h; a.msq = p->mask_stride_q;
  a.ssb = p->score_stride_b; a.ssh = p->score_stride_h; a.ssq = p->score_stride_q;
  a.B = p->batch; a.Tq = p->seqlen_q; a.Tk = p->seqlen_k; a.Hq = p->heads_q; a.Hk = p->heads_k;
  a.G = p->heads_q / p->heads_k;
  const int kb = kv_block_keys(p);
  a.nkt = (p->seqlen_k + kb - 1) / kb;
  const int dq_rows_rc = p->head_dim > 128 ? fa::dq_wide_block_rows() : fa::dq_block_rows();
  a.nqt = (p->seqlen_q + dq_rows_rc - 1) / dq_rows_rc;
  a.bk0 = 0;
  a.nbk = p->batch * p->heads_k;
  a.q32_lo = 0;
  a.q32_hi = (p->seqlen_q + 31) / 32;
  a.acc_mode = 0;
  a.sp0 = 0;
  a.nsp = split;
  a.g0 = 0;
  a.ng = a.G;
  a.ds_p0 = 0;
  a.split = split;
  a.do_dq = dq_atomics(p) ? 1 : 0;
  a.dq_split = dq_split_of(p);
  a.scale = p->scale;
  float sl2f;
  fill_scales(p->scale, &sl2f, &a.qsign, &a.zero_scale, &a.scale_log2);
  // dS tiles of the deterministic path
  a.nq32 = (p->seqlen_q + 31) / 32;
  a.nk32 = (p->seqlen_k + 31) / 32;
  a.ds = ds_elems(p) > 0 ? p->ds_tiles : nullptr;
  a.ds_plane = fa::ds_row(a.nq32, a.nk32, p->is_causal != 0);
  if (p->mask) {
    a.mws = (const char*)p->mask_ws;
    a.ml = layout_of(p->batch, p->heads_q, p->seqlen_q, p->seqlen_k, p->mask_stride_b, p->mask_stride_h);
  }
  return a;
}

int fa_bwd(const FaBwdParams* p) {
  if (!p) return fail(FA_ERR_NULL, "params is NULL");
  const int split = choose_split(p);
  int st = check_bwd(p, split);
  if (st) return st;
  const hipStream_t s = (hipStream_t)p->stream;
  const fa::BwdArgs a = bwd_args(p, split);
  const bool causal = p->is_causal != 0;

  if (p->head_dim > 128) {
    // head dim 256: dV and dK launches here, dQ (recomputed) in fa_bwd_finalize
    if ((st = launch_status(fa::launch_bwd_kv_wide(a, p->dtype, causal, s), "dkdv"))) return st;
  } else if (!a.ds || ds_slices(p) == 1) {
    // pipelined dK/dV (+ dS tiles when the plan has them) here, dQ in fa_bwd_finalize
    if ((st = launch_status(fa::launch_bwd_dkdv2(a, p->head_dim, p->dtype, causal, s), "dkdv"))) return st;
  } else if (std::vector<int> rb; row_ranges(p, &rb) > 0) {
    // row ranges: dK/dV of every unit over each range's rows (adding to fp32
    // sums that the first range writes and the last turns into dK/dV), then
    // dQ of those rows from the range's tiles (same stream: a range's tiles
    // are consumed before the next range overwrites them)
    const int nr = (int)rb.size() - 1;
    const int64_t nk32 = a.nk32;
    for (int r = 0; r < nr; ++r) {
      fa::BwdArgs k = a;
      k.q32_lo = rb[r];
      k.q32_hi = rb[r + 1];
      // one sum (split 1): the last range writes dK/dV; slabs (split > 1):
      // fa_bwd_finalize sums them
      k.acc_mode = r == 0 ? 1 : (r + 1 == nr && split == 1 ? 3 : 2);
      k.ds_plane = fa::ds_row(k.q32_hi, nk32, causal) - fa::ds_row(k.q32_lo, nk32, causal);
      if ((st = launch_status(fa::launch_bwd_dkdv2(k, p->head_dim, p->dtype, causal, s), "dkdv"))) return st;
      fa::BwdArgs q = k;
      q.acc_mode = 0;
      const int rows = std::min(p->seqlen_q, 32 * k.q32_hi) - 32 * k.q32_lo;
      // 512-row blocks (8 waves sharing each K tile) when they still give every CU one
      const bool wide = p->head_dim == 128 && !p->score &&
                        (int64_t)p->batch * p->heads_q * (rows / fa::kDqDsRowsWide) >= kCus;
      q.dq_rows = wide ? fa::kDqDsRowsWide : fa::kDqDsRows;
      q.nqt = (rows + q.dq_rows - 1) / q.dq_rows;
      if ((st = launch_status(fa::launch_bwd_dq_ds(q, p->head_dim, p->dtype, causal, s), "dq"))) return st;
    }
  } else if (int pper = 0, ps = part_split(p, &pper); ps > 0) {
    // parts of each unit's head group: per slice of parts, the dK/dV launch
    // writing those parts' fp32 slabs, then the dQ launch of their heads
    const int units = p->batch * p->heads_k, G = p->heads_q / p->heads_k, gsz = G / ps;
    for (int u = 0; u < units; ++u)
      for (int s0 = 0; s0 < ps; s0 += pper) {
        fa::BwdArgs k = a;
        k.bk0 = u;
        k.nbk = 1;
        k.sp0 = s0;
        k.nsp = std::min(pper, ps - s0);
        k.ds_p0 = (int64_t)u * G + (int64_t)s0 * gsz;
        if ((st = launch_status(fa::launch_bwd_dkdv2(k, p->head_dim, p->dtype, causal, s), "dkdv"))) return st;
        fa::BwdArgs q = k;
        q.g0 = s0 * gsz;
        q.ng = k.nsp * gsz;
        q.dq_rows = fa::kDqDsRows;
        q.nqt = (p->seqlen_q + q.dq_rows - 1) / q.dq_rows;
        if ((st = launch_status(fa::launch_bwd_dq_ds(q, p->head_dim, p->dtype, causal, s), "dq"))) return st;
      }
  } else {
    // the workspace holds a slice of (batch, kv-head) units: dK/dV and then
    // dQ of each slice (same stream, so a slice's tiles are consumed before
    // the next slice overwrites them)
    const int per = (int)ds_slice_units(p), units = p->batch * p->heads_k;
    fa::BwdArgs q = a;
    q.dq_rows = dq_rows(p);
    q.nqt = (p->seqlen_q + q.dq_rows - 1) / q.dq_rows;
    for (int u0 = 0; u0 < units; u0 += per) {
      fa::BwdArgs k = a;
      k.bk0 = q.bk0 = u0;
      k.nbk = q.nbk = std::min(per, units - u0);
      k.ds_p0 = q.ds_p0 = (int64_t)u0 * a.G;
      if ((st = launch_status(fa::launch_bwd_dkdv2(k, p->head_dim, p->dtype, causal, s), "dkdv"))) return st;
      if ((st = launch_status(fa::launch_bwd_dq_ds(q, p->head_dim, p->dtype, causal, s), "dq"))) return st;
    }
  }
  return FA_OK;
}

int fa_bwd_finalize(const FaBwdParams* p) {
  if (!p) return fail(FA_ERR_NULL, "params is NULL");
  const int split = choose_split(p);
  int st = check_bwd(p, split);
  if (st) return st;
  const hipStream_t s = (hipStream_t)p->stream;
  {
    // dQ = scale dS K from the tiles fa_bwd stored (written, or added over key
    // ranges with fp32 atomics), or recomputed
    fa::BwdArgs a = bwd_args(p, split);
    const bool causal = p->is_causal != 0;
    if (a.ds) {
      // sliced: fa_bwd already ran the dQ kernel per slice
      a.dq_rows = dq_rows(p);
      a.nqt = (p->seqlen_q + a.dq_rows - 1) / a.dq_rows;
      if (ds_slices(p) == 1 && (st = launch_status(fa::launch_bwd_dq_ds(a, p->head_dim, p->dtype, causal, s), "dq")))
        return st;
    } else if (p->head_dim > 128) {
      if ((st = launch_status(fa::launch_bwd_dq_wide(a, p->dtype, causal, s), "dq"))) return st;
    } else {
      if ((st = launch_status(fa::launch_bwd_dq(a, p->head_dim, p->dtype, causal, s), "dq"))) return st;
    }
  }
  if (dq_atomics(p)) {
    // dq_accum is head-major [B, Hq, Tq, D]
    const int64_t D = p->head_dim, Tq = p->seqlen_q, Hq = p->heads_q;
    fa::CvtArgs c{p->dq_accum, p->dq, p->dq_stride_b, p->dq_stride_t, p->dq_stride_h,
                  p->batch, p->seqlen_q, p->heads_q, p->head_dim, 1, 0, Hq * Tq * D, D, Tq * D};
    if ((st = launch_status(fa::launch_convert(c, p->dtype, s), "dq convert"))) return st;
  }
  if (split > 1) {
    // one slab per head-group part, summed in a fixed order
    const int nslab = split;
    const int64_t slab = (int64_t)p->batch * p->seqlen_k * p->heads_k * p->head_dim;
    const int64_t D = p->head_dim, Tk = p->seqlen_k, Hk = p->heads_k;
    fa::CvtArgs ck{p->dk_accum, p->dk, p->dk_stride_b, p->dk_stride_t, p->dk_stride_h,
                   p->batch, p->seqlen_k, p->heads_k, p->head_dim, nslab, slab, Tk * Hk * D, Hk * D, D};
    if ((st = launch_status(fa::launch_convert(ck, p->dtype, s), "dk convert"))) return st;
    fa::CvtArgs cv{p->dv_accum, p->dv, p->dv_stride_b, p->dv_stride_t, p->dv_stride_h,
                   p->batch, p->seqlen_k, p->heads_k, p->head_dim, nslab, slab, Tk * Hk * D, Hk * D, D};
    if ((st = launch_status(fa::launch_convert(cv, p->dtype, s), "dv convert"))) return st;
  }
  return FA_OK;
}

// Allocation-free backward: the deterministic route with dQ recomputed and
// dK/dV written directly (no dS tiles, no fp32 accumulators), with Delta, the
// backward LSE and the dead-row flags in the library's device scratch
// (fa_noalloc.hip) instead of caller workspaces.
int fa_bwd_noalloc(const FaBwdParams* p) {
  if (!p) return fail(FA_ERR_NULL, "params is NULL");
  int st = check_dims(p->batch, p->seqlen_q, p->seqlen_k, p->heads_q, p->heads_k, p->head_dim, p->dtype, p->scale);
  if (st) return st;
  const int64_t rows = (int64_t)p->batch * p->heads_q * p->seqlen_q;
  const int64_t flag_off = fa::align256(2 * rows * (int64_t)sizeof(float));
  const int64_t need = flag_off + (int64_t)p->batch * p->heads_k * (int64_t)sizeof(int32_t);
  const int64_t cap = fa::noalloc_scratch_bytes();
  if (need > cap)
    return fail(FA_ERR_WORKSPACE,
                "fa_bwd_noalloc needs %lld bytes of device scratch (8 B per query row of every head, 4 B per "
                "(batch, kv-head)); it holds %lld (B*Hq*Tq up to about %lld): use fa_bwd with workspaces",
                (long long)need, (long long)cap, (long long)(cap / 8));
  // validate everything with stand-in workspace addresses before any HIP call
  FaBwdParams q = *p;
  q.dq_accum = q.dk_accum = q.dv_accum = nullptr;
  q.ds_tiles = nullptr;
  q.ds_limit_bytes = -1;   // no dS tiles: dQ is recomputed
  q.atomic_dq = 0;
  q.kv_split = 1;          // dK/dV written by the kernel, no fp32 slabs
  q.delta = (float*)(uintptr_t)256;
  q.dead_flags = (int32_t*)(uintptr_t)256;
  if ((st = check_bwd(&q, 1))) return st;
  void* base = nullptr;
  const hipError_t e = fa::scratch_device_ptr(&base);
  if (e != hipSuccess) return fail(FA_ERR_LAUNCH, "fa_bwd_noalloc: device scratch lookup failed: %s", hipGetErrorString(e));
  q.delta = (float*)base;
  q.dead_flags = (int32_t*)((char*)base + flag_off);
  if ((st = launch_status(fa::launch_fill_i32(q.dead_flags, (int64_t)p->batch * p->heads_k, 0, (hipStream_t)p->stream),
                          "fa_bwd_noalloc flag clear")))
    return st;
  if ((st = fa_bwd_preprocess(&q))) return st;
  if ((st = fa_bwd(&q))) return st;
  return fa_bwd_finalize(&q);
}

}  // extern "C"
