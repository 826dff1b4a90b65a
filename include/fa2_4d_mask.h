/*
 * fa2_4d_mask.h -- C ABI of the MI355X (gfx950) FlashAttention-2 forward and
 * backward with optional 4D bool keep-mask and 4D fp32 score.
 *
 * The library (libfa2_4d_mask.so) replaces the four TileLang JIT kernels of
 * the reference (python/fa2.py) and is called by the host mirror of the
 * reference's autograd Function (tilelang_fa2_4d_mask/fa2.py in this build).
 *
 * Conventions
 *  - All pointers are device pointers; the caller owns every buffer (outputs
 *    and workspaces).  Nothing here allocates device memory.
 *  - Strides are in ELEMENTS.  The head dimension (D) of Q/K/V/O/dO/dQ/dK/dV
 *    must be contiguous (stride 1); batch/time/head strides are free, so BHSD
 *    views over BTHD storage and BHSD-contiguous tensors both work uncopied.
 *  - Mask is bool (1 byte, 0 = drop, nonzero = keep) and Score is fp32, both
 *    logically [B, Hq, Tq, Tk] with the key dimension contiguous; a batch or
 *    head stride of 0 broadcasts (e.g. a [B, 1, Tq, Tk] mask).
 *  - A mask is first turned into a prepared-mask workspace by fa_mask_prepare
 *    (bits, 32x32 block states, lists of live tiles); fa_fwd and fa_bwd take
 *    that workspace (mask_ws) beside the mask and skip tiles without a kept
 *    entry.
 *  - LSE is fp32 [B, Hq, Tq] contiguous, base-2 log-sum-exp of the scaled
 *    logits; +inf marks a row with no kept key.  Internal fwd->bwd contract.
 *  - Every entry point validates its arguments before touching the GPU and
 *    returns 0 when the kernels were enqueued on `stream`, or a nonzero
 *    FA_ERR_* code with nothing launched; fa_last_error() then describes it.
 *    Launches are asynchronous, never synchronise, and keep no state between
 *    calls, so they can be captured into a HIP graph.
 */
#ifndef FA2_4D_MASK_H
#define FA2_4D_MASK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 6

enum FaDtype { FA_DTYPE_BF16 = 0, FA_DTYPE_FP16 = 1 };

enum FaStatus {
  FA_OK = 0,
  FA_ERR_NULL = 1,        /* a required pointer is NULL */
  FA_ERR_SHAPE = 2,       /* non-positive size, Hq % Hk != 0, ... */
  FA_ERR_HEAD_DIM = 3,    /* head_dim not supported by a kernel instance (64, 128, 256) */
  FA_ERR_DTYPE = 4,       /* dtype not FA_DTYPE_BF16 / FA_DTYPE_FP16 */
  FA_ERR_STRIDE = 5,      /* head-dim stride != 1 or misaligned base */
  FA_ERR_SCALE = 6,       /* scale is NaN or infinite */
  FA_ERR_LAUNCH = 7,      /* the HIP runtime refused the launch */
  FA_ERR_WORKSPACE = 8    /* a workspace required by the chosen plan is missing */
};

/* Forward problem: O = softmax(((Q K^T + Score) * scale) masked) V, plus LSE. */
typedef struct FaFwdParams {
  const void* q;                 /* [B, Tq, Hq, D] (by strides), dtype */
  const void* k;                 /* [B, Tk, Hk, D] */
  const void* v;                 /* [B, Tk, Hk, D] */
  void* o;                       /* [B, Tq, Hq, D] output, dtype */
  float* lse;                    /* [B, Hq, Tq] fp32 output, contiguous */
  const uint8_t* mask;           /* optional, NULL if absent */
  const float* score;            /* optional, NULL if absent */
  int64_t q_stride_b, q_stride_t, q_stride_h;
  int64_t k_stride_b, k_stride_t, k_stride_h;
  int64_t v_stride_b, v_stride_t, v_stride_h;
  int64_t o_stride_b, o_stride_t, o_stride_h;
  int64_t mask_stride_b, mask_stride_h, mask_stride_q;
  int64_t score_stride_b, score_stride_h, score_stride_q;
  int32_t batch, seqlen_q, seqlen_k, heads_q, heads_k, head_dim;
  float scale;                   /* softmax scale applied after adding Score */
  int32_t is_causal;             /* keep j <= i (top-left aligned) */
  int32_t dtype;                 /* enum FaDtype */
  void* stream;                  /* hipStream_t; NULL = default stream */
  const void* mask_ws;           /* prepared mask (fa_mask_prepare of this mask); required with a mask */
  void* o_lo;                    /* optional [B, Tq, Hq, D] dtype output, written with a mask or a score only:
                                    O's rounding residual (O in fp32 minus O as stored, rounded to dtype),
                                    for fa_bwd_preprocess; NULL = not written */
  int64_t o_lo_stride_b, o_lo_stride_t, o_lo_stride_h;
} FaFwdParams;

/* Backward problem.  Reuses the forward's inputs plus O, LSE and dO. */
typedef struct FaBwdParams {
  const void* q; const void* k; const void* v;
  const void* o;                 /* forward output */
  const void* dout;              /* gradient of O, [B, Tq, Hq, D] by strides */
  const float* lse;              /* [B, Hq, Tq] from fa_fwd */
  float* delta;                  /* workspace [2, B, Hq, Tq] fp32, written by fa_bwd_preprocess: Delta, then
                                    the LSE the backward kernels read (the forward's, except -inf for a
                                    row whose kept keys all have a -inf logit) */
  int32_t* dead_flags;           /* workspace [B * Hk] int32, zeroed by the caller */
  const uint8_t* mask; const float* score;
  float* dq_accum;               /* workspace [B, Hq, Tq, D] fp32 contiguous, head-major (atomic dQ) */
  float* dk_accum;               /* workspace of plan.dkv_accum_elems fp32, when that is > 0 (head-group
                                    split slabs, or the running sums over ranges of query rows) */
  float* dv_accum;               /* idem */
  void* dq; void* dk; void* dv;  /* outputs, dtype, strided like q/k/v */
  int64_t q_stride_b, q_stride_t, q_stride_h;
  int64_t k_stride_b, k_stride_t, k_stride_h;
  int64_t v_stride_b, v_stride_t, v_stride_h;
  int64_t o_stride_b, o_stride_t, o_stride_h;
  int64_t do_stride_b, do_stride_t, do_stride_h;
  int64_t dq_stride_b, dq_stride_t, dq_stride_h;
  int64_t dk_stride_b, dk_stride_t, dk_stride_h;
  int64_t dv_stride_b, dv_stride_t, dv_stride_h;
  int64_t mask_stride_b, mask_stride_h, mask_stride_q;
  int64_t score_stride_b, score_stride_h, score_stride_q;
  int32_t batch, seqlen_q, seqlen_k, heads_q, heads_k, head_dim;
  float scale;
  int32_t is_causal;
  int32_t atomic_dq;             /* 1: fp32 atomic dQ (default); 0: deterministic dQ kernel */
  int32_t kv_split;              /* query-head-group split of the dK/dV kernel; 0 = let fa_bwd_plan choose */
  int32_t dtype;
  void* stream;
  void* ds_tiles;                /* workspace of plan.ds_elems 16-bit values (deterministic path), else unused */
  int64_t ds_limit_bytes;        /* largest dS workspace the caller accepts; 0 = 4 GiB, < 0 = none
                                    (below the whole need: the backward runs in slices of units, or
                                    in ranges of query rows; see FaBwdPlan.ds_elems) */
  const void* mask_ws;           /* prepared mask, as for fa_fwd; required with a mask */
  const void* o_lo;              /* optional: the o_lo fa_fwd wrote; Delta = sum_d dO (O + o_lo) */
  int64_t o_lo_stride_b, o_lo_stride_t, o_lo_stride_h;
  int64_t ds_tiles_elems;        /* 16-bit elements the caller allocated at ds_tiles; when ds_tiles is given
                                    it must be at least plan.ds_elems of this problem (which depends on
                                    whether a mask or a score is given), else FA_ERR_WORKSPACE */
} FaBwdParams;

/* Mask preparation: the bool mask of a problem turned into the workspace the
 * attention kernels read (the mask as bits, row-major and transposed; the
 * state of every 32x32 block; per work unit of each kernel the list of tiles
 * holding a kept entry, causality included).  The workspace depends on the
 * mask's contents, its batch/head broadcast (stride 0), the sizes and
 * is_causal, and serves every fa_fwd / fa_bwd call with those. */
typedef struct FaMaskParams {
  const uint8_t* mask;           /* logical [B, Hq, Tq, Tk] by strides, key axis contiguous */
  int64_t mask_stride_b, mask_stride_h, mask_stride_q;
  int32_t batch, seqlen_q, seqlen_k, heads_q;
  int32_t is_causal;
  void* workspace;               /* fa_mask_plan bytes, 256-byte aligned, written by fa_mask_prepare */
  void* stream;
} FaMaskParams;

/* What fa_bwd will do for a problem, so the caller can size workspaces. */
typedef struct FaBwdPlan {
  int32_t kv_split;              /* >1: dK/dV of each head-group part go to fp32 dk_accum/dv_accum slabs,
                                    summed by fa_bwd_finalize */
  int32_t needs_dq_accum;        /* 1 if dq_accum is used: dQ added with fp32 atomics (atomic_dq = 1 and
                                    dq_split > 1); else dQ is written directly */
  int64_t dq_accum_elems;        /* B*Tq*Hq*D when used, else 0 */
  int64_t dkv_accum_elems;       /* kv_split > 1: B*Tk*Hk*D per slab (kv_split slabs); ranges of query
                                    rows (ds_elems) at kv_split 1: B*Tk*Hk*D, the running sums; written
                                    by the kernels (first range), never read before; else 0 */
  int64_t ds_elems;              /* size of ds_tiles: 16-bit dS of every stored 32x32 block of all
                                    (batch, kv-head) units when they fit ds_limit_bytes; else of a slice
                                    of as many units as fit (nearly equal slices, run one after the
                                    other); else, without a mask, of the largest range of query rows
                                    (512-row multiples, every unit; fa_bwd runs the ranges one after
                                    the other and sums dK/dV across them in dk_accum/dv_accum) -- causal
                                    problems without a mask take the ranges whenever they do not fit
                                    at once; with a mask, of as many one-head parts of a unit's group
                                    as fit (kv_split = the group size, one slab per part).  0 when
                                    not even one unit, 512-row range, nor (with a mask) plane fits:
                                    dQ is then recomputed, in both modes */
  int32_t dkv_accum_zeroed;      /* 1: dk_accum/dv_accum must be zeroed by the caller (0 in this ABI) */
  int32_t dq_split;              /* atomic_dq = 1 with dS tiles: key ranges whose dQ partials are added
                                    (2-8) when the 256-row query blocks are fewer than the CUs; 1: each
                                    block writes its rows, no atomics (as atomic_dq = 0) */
} FaBwdPlan;

/* Size in bytes of the prepared-mask workspace for *p (no launch, no GPU access). */
int fa_mask_plan(const FaMaskParams* p, int64_t* workspace_bytes);

/* Writes the prepared-mask workspace.  Replaces the per-tile mask loads of the
 * reference kernels (python/fa2.py:107-114, 261-280, 385-404) with one pass over the
 * mask; the reference materialises the broadcast mask instead
 * (python/modeling_attention.py:48-59).  Must precede the fa_fwd / fa_bwd calls that
 * read the workspace on the same stream. */
int fa_mask_prepare(const FaMaskParams* p);

/* Forward.  Replaces the reference's `flash_attention_fwd_with_4d_mask`
 * (python/fa2.py:22-139) as launched by `_flash_attention_with_4d_mask.forward`
 * (python/fa2.py:474-478).  Writes O and LSE (and o_lo when given, with a mask or
 * a score).  With a mask or a score the probabilities enter O += P V as two 16-bit
 * halves, P rounded and its rounding residual (the reference rounds P once,
 * python/fa2.py:128-129); the backward does the same for P and dS. */
int fa_fwd(const FaFwdParams* p);

/* Backward preprocess.  Replaces `bwd_preprocess` (python/fa2.py:142-179, launched at
 * python/fa2.py:509-513): delta[b,h,i] = sum_d O*dO in fp32; additionally zeroes the
 * dq_accum rows (when the plan uses it), and for rows whose LSE is +inf (every kept
 * logit -inf) zeroes delta and raises dead_flags[b*Hk+kvh].  Such a row gets the
 * eager reference's gradients (benchmark/precision_check.py:158-174 under autograd):
 * with no kept key (mask, causality) a zero dQ row; with kept keys whose logits are
 * all -inf (a -inf score) a NaN dQ row and NaN dK rows at those keys; dV of the
 * kv-head NaN in both cases. */
int fa_bwd_preprocess(const FaBwdParams* p);

/* Backward main pass.  Replaces `flash_attention_bwd_with_4d_mask_atomic`
 * (python/fa2.py:181-302, launched at :530-534) when atomic_dq = 1 and
 * `flash_attention_bwd_with_4d_mask_reduce` (python/fa2.py:305-426, launched at
 * :543-547) when atomic_dq = 0.  With plan.ds_elems > 0 (both modes): the dK/dV
 * kernel, writing dK/dV in dtype (kv_split = 1) or per-split fp32 slabs, and
 * storing dS into ds_tiles for fa_bwd_finalize (when ds_tiles holds a slice of the
 * (batch, kv-head) units, fa_bwd runs the dK/dV and the dQ kernel per slice and
 * fa_bwd_finalize only converts; likewise over ranges of query rows, or parts of
 * the head groups).  With plan.ds_elems = 0 (both modes): the dK/dV kernel only.
 * Must follow fa_bwd_preprocess on the same stream. */
int fa_bwd(const FaBwdParams* p);

/* Backward finalisation.  dQ: from ds_tiles, dQ = scale dS K, written in dtype
 * (atomic_dq = 0, or plan.dq_split = 1) or added as fp32 partials over
 * plan.dq_split key ranges into dq_accum with atomics and converted (atomic_dq = 1,
 * plan.dq_split > 1); without ds_tiles,
 * recomputed from S, P and dP (both modes).  dk, dv from dk_accum/dv_accum when
 * kv_split > 1.  Replaces the casts of python/fa2.py:535-536, the group sum of
 * python/fa2.py:548-549 and autograd's cast of the fp32 dQ the reference returns
 * (python/fa2.py:527, 556); the dS-based dQ replaces the per-64-key dQ atomics of
 * python/fa2.py:295-297, 420-421.  Must follow fa_bwd on the same stream. */
int fa_bwd_finalize(const FaBwdParams* p);

/* Backward without any workspace from the caller and without allocating.  No
 * counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * Same problem, inputs, outputs and results as fa_bwd_preprocess + fa_bwd +
 * fa_bwd_finalize with atomic_dq = 0 and no dS workspace (ds_limit_bytes < 0):
 * dK/dV from the dK/dV kernel, dQ recomputed, deterministic.  Ignores delta,
 * dead_flags, dq_accum, dk_accum, dv_accum, ds_tiles, ds_limit_bytes, atomic_dq
 * and kv_split.  Delta, the backward LSE and the dead-row flags live in a 16 MiB
 * device array of the library, one per GPU, held until the process ends: a
 * problem needs 8 bytes per query row of every head plus 4 per (batch, kv-head),
 * i.e. B*Hq*Tq up to about 2 million rows; larger ones return FA_ERR_WORKSPACE.
 * Calls on one GPU share that array: calls that overlap on one GPU (other
 * streams, unordered host threads) race.  A mask still needs its prepared
 * workspace (mask_ws, the one the forward used).  The current device must be the
 * stream's. */
int fa_bwd_noalloc(const FaBwdParams* p);

/* Fills *plan for the problem in *p (no launch, no GPU access): sizes, head dim,
 * dtype, causality, atomic_dq, kv_split, ds_limit_bytes and whether mask / score
 * are non-NULL (with either, every dS block is stored as a pair of tiles). */
int fa_bwd_plan(const FaBwdParams* p, FaBwdPlan* plan);

/* Human-readable description of the last nonzero status on the calling thread. */
const char* fa_last_error(void);

/* FA_ABI_VERSION of the library. */
int fa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FA2_4D_MASK_H */
