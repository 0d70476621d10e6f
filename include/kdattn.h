/*
 * kdattn.h -- C ABI of the MI355X (gfx950) hierarchical-mask flash attention.
 *
 * Drop-in device boundary for KernelDev's attention hot path.  The Python
 * package kerneldev_amd binds these entry points with ctypes behind the same
 * flash_attention() signature as the reference (original_kernel.py:2096-2112).
 *
 * Conventions
 *   - Every function returns an int status: KD_OK (0) or a negative KD_ERR_*;
 *     kd_last_error_string() describes the last failure on the calling thread.
 *     No C++ exception crosses this boundary.
 *   - The caller owns all device memory: inputs, outputs and workspaces are
 *     plain device pointers.  The library never allocates or frees device
 *     memory and keeps no state between calls apart from its code objects.
 *   - Work is enqueued asynchronously on `stream` (a hipStream_t passed as
 *     void*; NULL is the default stream).  No call synchronises the host.
 *   - Tensors [B, H, T, D] are given by a base pointer and element strides for
 *     (b, h, t); the d stride must be 1, base pointers 16-byte aligned, the
 *     (b, h, t) strides multiples of 8 elements, the t stride >= D and
 *     T * t_stride * element size < 2^31 bytes.
 *   - Head dims 16, 32, 64, 128, 256 (original_kernel.py:1720).  bf16 / fp16
 *     run on the MFMA kernels at every head dim (16 and 32 on the D = 64
 *     kernels, which read the columns past D as zeros and store only the D
 *     real ones; dqk_signs at 64, 128 only; fp8 scores at 64, 128, 256 for bf16); fp32 inputs
 *     on the fp32 MFMA kernels at every head dim (16 on the D = 32 kernels,
 *     the same way).  fp32 inputs get no fp8 scores and no dqk_signs,
 *     and precision is always full fp32 for them.  (The Python layer runs fp32 inputs at precision "tf32"
 *     and D = 16, 32 as bf16 operands of three times the head dim on the
 *     16-bit MFMA kernels instead, with dq_lo / dk_lo / dv_lo below.)
 *   - LSE is stored in log2 units (LSE2 = log2 sum_j exp2(S_ij * sm_scale *
 *     log2 e)), as the reference stores it (original_kernel.py:603-604).
 *     Fully masked rows get O = 0, LSE = -inf and zero gradients.
 */
#ifndef KDATTN_H
#define KDATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KD_OK 0
#define KD_ERR_INVALID -1     /* bad argument: shape, stride, pointer, alignment */
#define KD_ERR_UNSUPPORTED -2 /* head dim / dtype / mode not built */
#define KD_ERR_LAUNCH -3      /* HIP launch error */

/* element dtypes */
#define KD_BF16 0
#define KD_F16 1
#define KD_F32 2 /* attention only: computed in fp32 (fp32 MFMA at every head dim) */
/* arithmetic of the softmax weights P and the score gradients dS inside the
 * attention kernels (kd_attn_args.precision) */
#define KD_PREC_SPLIT 0  /* P and dS enter their products (P V, dV, dQ, dK) as a 16-bit pair
                            hi + lo, ~16 significant bits (default) */
#define KD_PREC_SINGLE 1 /* P and dS rounded once to the input type (8 significant bits for
                            bf16, as the reference's forward rounds P to V's dtype) */
#define KD_PREC_SPLIT3 2 /* P and dS enter their products as a 16-bit triple hi + mid + lo, ~24
                            significant bits (bf16), as the reference's fp32 backward dots take
                            them at precision "ieee"; the residual outputs o_lo, dq_lo, dk_lo and
                            dv_lo are then fp32, so that o + o_lo (etc.) carry fp32 precision and
                            the backward's Delta sees O to it.  Not with fp8 scores. */
/* span_id index dtypes */
#define KD_I64 0
#define KD_I32 1
/* mask modes -- which branch of original_kernel.py:401, :478-517 applies */
#define KD_MODE_FORMULA 0 /* any metadata given, or attention_mask given */
#define KD_MODE_CAUSAL 1  /* no metadata, causal=True:  i >= j  (:512-513) */
#define KD_MODE_ALL 2     /* no metadata, causal=False: all True (:514-515) */

/* Mask metadata, as the reference's forward adapter receives it
 * (original_kernel.py:1697-1715: lens, in_span, span_id, is_prefix). */
typedef struct kd_meta_args {
  const uint8_t *in_span;   /* bool [B, T] or NULL */
  int64_t in_span_strides[2];
  const void *span_id;      /* int64 or int32 [B, T] or NULL */
  int64_t span_id_strides[2];
  int32_t span_id_dtype;    /* KD_I64 / KD_I32 */
  int32_t mode;             /* KD_MODE_* */
  const uint8_t *is_prefix; /* bool [B, T] or NULL */
  int64_t is_prefix_strides[2];
  const int32_t *lens;      /* int32 [B] or NULL */
  int64_t lens_stride;
  int32_t B, T, D;
  int32_t pad_;
} kd_meta_args;

/* Token rows for kd_plan_build_tokens: ids of data_builder.py:44-52
 * ([PAD]=0, [CLS]=1, [MASK]=2, [SPAN]=3, [ES]=4, [MASKQ]=5, bytes + 6). */
#define KD_RULE_COLLATE 0   /* data_builder.py:603-643: [SPAN]..[ES] inclusive, first [MASKQ] -> -1 */
#define KD_RULE_FALLBACK 1  /* model.py:209-240: [ES] outside its span, every [MASKQ] -> -1 */
#define KD_RULE_TEACHER 2   /* train_loop.py:406-435: prefix only */
typedef struct kd_token_args {
  const void *tokens;       /* int64 or int32 [B, T] */
  int64_t tokens_strides[2];
  int32_t tokens_dtype;     /* KD_I64 / KD_I32 */
  int32_t rule;             /* KD_RULE_* */
  const int32_t *lens;      /* int32 [B] or NULL */
  int64_t lens_stride;
  int32_t B, T, D;
  int32_t pad_;
} kd_token_args;

/* Attention operands (forward and backward share one struct). */
typedef struct kd_attn_args {
  const void *q, *k, *v;        /* [B, H, T, D] */
  int64_t q_strides[3], k_strides[3], v_strides[3];
  void *o;                      /* [B, H, T, D] output (fwd) / input (bwd) */
  int64_t o_strides[3];
  float *lse;                   /* [B, H, T] fp32, contiguous */
  const void *dout;             /* [B, H, T, D] (bwd) */
  int64_t do_strides[3];
  void *dq, *dk, *dv;           /* [B, H, T, D] (bwd) */
  int64_t dq_strides[3], dk_strides[3], dv_strides[3];
  float *delta;                 /* fp32 workspace of 2 * B*H*T (bwd): -Delta [B, H, T],
                                   then -LSE / c [B, H, T] with c the score scale (sm_scale log2 e, times
                                   q_scale k_scale with fp8 scores; -inf for fully masked rows) */
  void *o_lo;                   /* optional contiguous [B, H, T, D], dtype of o (bf16 /
                                   fp16 only; NULL with fp32 inputs), fp32 at precision
                                   KD_PREC_SPLIT3: the forward writes O_fp32 - O there, the
                                   backward's Delta reads it; NULL to skip */
  const uint8_t *q8, *k8;       /* optional fp8 e4m3 copies of q and k, contiguous
                                   [B, H, T, D] (kd_quant_fp8): when both are given, S = Q K^T
                                   is computed from them on fp8 MFMA, times q_scale * k_scale */
  const float *q_scale, *k_scale; /* [B, H] dequantisation scales of q8 / k8 */
  const float *dqk_signs;       /* optional [D] of +1 / -1 (bwd): q and k are rotated inputs
                                   Q R, K R with R = diag(signs) H_D / sqrt(D) (kd_hadamard), and
                                   dQ, dK are returned for the unrotated Q, K, i.e. times R^T,
                                   applied in the kernels' epilogues; NULL: dQ, dK as computed */
  void *dq_lo, *dk_lo, *dv_lo;  /* optional contiguous [B, H, T, D] of the 16-bit dtype (fp32 at
                                   precision KD_PREC_SPLIT3) (bwd): the
                                   rounding residuals dQ_fp32 - dQ (etc.), so that dq + dq_lo carries
                                   the gradient to ~16 significant bits (as o_lo does for O); NULL to
                                   skip; not with dqk_signs or fp32 inputs */
  int32_t B, H, T, D;
  int32_t dtype;                /* KD_BF16 / KD_F16 / KD_F32 */
  float sm_scale;
  int32_t precision;            /* KD_PREC_SPLIT (0, default) / KD_PREC_SINGLE / KD_PREC_SPLIT3 */
  int32_t pad_;
} kd_attn_args;

/* Walsh-Hadamard rotation of [B, H, T, D] rows (incoherent processing). */
typedef struct kd_rot_args {
  const void *x;                /* [B, H, T, D] input */
  int64_t x_strides[3];
  void *y;                      /* [B, H, T, D] output (may not alias x) */
  int64_t y_strides[3];
  const float *signs;           /* [D] of +1 / -1 */
  float *amax;                  /* optional [B, H]: max |y| is atomically max-ed in; zero it first */
  int32_t B, H, T, D;
  int32_t dtype;                /* KD_BF16 / KD_F16 */
  int32_t inverse;              /* 0: y = x R;  1: y = x R^T */
} kd_rot_args;

/* Per-(b, h) fp8 e4m3 quantisation: y = e4m3(clamp(x * fp32(448 / amax), +-448)),
 * round to nearest even, scale = amax / 448 (amax == 0: both factors 1). */
typedef struct kd_quant_args {
  const void *x;                /* [B, H, T, D] bf16 / fp16 */
  int64_t x_strides[3];
  uint8_t *y;                   /* contiguous [B, H, T, D] e4m3 bytes */
  const float *amax;            /* [B, H] max |x| (kd_hadamard can produce it) */
  float *scale;                 /* [B, H] output: amax / 448 */
  int32_t B, H, T, D;
  int32_t dtype;
  int32_t pad_;
} kd_quant_args;

/* Cocktail-party head (model.py:263-298): per row, the hidden state at the
 * first [MASK] (h_ctx, zero if none) is scored against the mean hidden state
 * of each span's interior.  The j-th [SPAN] of a row pairs with the row's
 * j-th [ES] (the reference zips the two position lists, :287-291); the
 * interior is [pos([SPAN]_j) + 1, pos([ES]_j)), and a pair without a partner
 * or with an empty interior scores 0 (the reference's zero h_spans row,
 * :285, :292).  kd_span_scores fills the forward outputs; kd_span_scores_bwd
 * turns d scores into d h, reading the forward's outputs. */
typedef struct kd_span_args {
  const void *tokens;       /* int64 or int32 [B, T] (ids of data_builder.py:44-52) */
  int64_t tokens_strides[2];
  int32_t tokens_dtype;     /* KD_I64 / KD_I32 */
  int32_t dtype;            /* KD_BF16 / KD_F16: h and dh */
  const void *h;            /* [B, T, D] hidden states, unit d stride */
  int64_t h_strides[2];     /* (b, t) in elements */
  int32_t B, T, D;          /* D <= 65536 */
  int32_t n_spans;          /* score columns, 1 .. 8192; the reference's max_spans = the
                               largest per-row [SPAN] count (spans past n_spans are dropped) */
  float *scores;            /* out [B, n_spans] */
  float *h_ctx;             /* out [B, D] */
  float *h_spans;           /* out [B, n_spans, D] span means (0 where none) */
  int32_t *span_lo;         /* out [B, n_spans]: interior [lo, hi); lo == hi where none */
  int32_t *span_hi;
  int32_t *mask_pos;        /* out [B]: first [MASK] position or -1 */
  const float *dscores;     /* bwd in [B, n_spans] */
  void *dh;                 /* bwd out [B, T, D] (dtype), every element written */
  int64_t dh_strides[2];    /* (b, t) in elements, unit d stride */
} kd_span_args;

/* Library version (major*10000 + minor*100 + patch).  3.0.0: the plan's size
 * beside its pointer in every entry point that takes a plan.  3.1.0:
 * kd_plan_layout writes 20 offsets (the dK/dV work order added).  3.2.0:
 * kd_absmax added.  3.3.0: fp8 scores (q8 / k8) and kd_quant_fp8 at head
 * dim 256. */
int kd_version(void);

/* Message for the last non-zero status returned on this thread. */
const char *kd_last_error_string(void);

/* sizeof(kd_meta_args), sizeof(kd_attn_args): lets bindings check layouts. */
void kd_struct_sizes(size_t *meta, size_t *attn);
void kd_struct_sizes2(size_t *rot, size_t *quant);
void kd_struct_sizes3(size_t *tokens);

/* Every entry point that reads or writes a plan takes the plan's size in bytes
 * (plan_bytes) beside its pointer, and returns KD_ERR_INVALID, launching
 * nothing, when it is below kd_plan_bytes(B, T, D) of the call's shape: the
 * kernels index the plan by that layout.  The check is on the host, with no
 * device access and no synchronisation.
 *
 * Workspace ("plan") bytes for B sequences of length T at head dim D, and
 * the byte offsets of its sections (token codes, class map, per-tile allowed
 * counts, the forward / dQ / dK-dV work lists, the work orders).  offsets[]
 * receives 20 int64: codes, rep, cls, nnz, fwd_list, fwd_count, dq_list,
 * dq_count, dkdv_list, dkdv_count, nT, fwd_group, dq_group, dkdv_group,
 * n_fwd_blocks, n_dq_blocks, n_dkdv_blocks, fwd_order, dq_order, dkdv_order.
 * A list entry is (tile << 8) | the class of group member r in bits 2r..2r+1.
 * A work order (u32 [B n]) lists the items b n + block of the forward, dQ or
 * dK/dV list by descending list length (equal lengths in ascending item
 * order); the forward, dQ and dK/dV kernels take each head's blocks in that
 * order.  The plan holds no
 * per-element masks (the kernels build PARTIAL tiles' masks from the codes),
 * so it takes O(B T + B nT^2) bytes.  Replaces the per-tile mask evaluation of
 * original_kernel.py:457-517 (the reference has no tile map). */
int64_t kd_plan_bytes(int32_t B, int32_t T, int32_t D);
int kd_plan_layout(int32_t B, int32_t T, int32_t D, int64_t *offsets);

/* Build the plan: token codes, 64x64 tile class map (0 empty / 1 partial /
 * 2 full, bit-exact against the dense mask), allowed-entry counts and the
 * per-block work lists.  Mask rules: original_kernel.py:478-517, with lens
 * (:299-303, :517) and the no-metadata fallbacks (:512-515). */
int kd_plan_build(const kd_meta_args *meta, void *plan, int64_t plan_bytes, void *stream);

/* The plan straight from token ids: is_prefix, in_span and span_id are derived
 * on the device by the chosen rule (written into the plan's own workspace) and
 * the plan is then built as kd_plan_build would from them.  Replaces the
 * per-token Python loops with host syncs at data_builder.py:603-643,
 * model.py:209-240 and train_loop.py:406-435 ahead of the mask evaluation. */
int kd_plan_build_tokens(const kd_token_args *t, void *plan, int64_t plan_bytes, void *stream);

/* Forward: O and LSE.  Replaces attention_forward_adapter's launch of
 * _flash_attn_fwd (original_kernel.py:1697-1778, kernel :279-626). */
int kd_attn_fwd(const kd_attn_args *a, const void *plan, int64_t plan_bytes, void *stream);

/* -Delta = -rowsum(O * dO) in fp32 into a->delta[0 : B*H*T], and -LSE / c
 * (the form kd_attn_bwd_dkdv starts its score accumulators from; -inf for
 * fully masked rows) into a->delta[B*H*T : 2*B*H*T].  Replaces
 * _flash_attn_bwd_precompute (original_kernel.py:649-710, launch :1829-1846).
 * kd_attn_bwd_dq reads the first half, kd_attn_bwd_dkdv both. */
int kd_attn_bwd_delta(const kd_attn_args *a, void *stream);

/* dQ from the saved LSE and Delta.  Replaces the dQ workers of
 * _flash_attn_bwd (original_kernel.py:1173-1336). */
int kd_attn_bwd_dq(const kd_attn_args *a, const void *plan, int64_t plan_bytes, void *stream);

/* dQ that computes Delta and the LSE copy itself (from a->o, a->o_lo, a->lse)
 * and stores both halves of a->delta for kd_attn_bwd_dkdv: the work of
 * _flash_attn_bwd_precompute (original_kernel.py:649-710) and of the dQ
 * workers (:1173-1336) in one pass. */
int kd_attn_bwd_dq_delta(const kd_attn_args *a, const void *plan, int64_t plan_bytes, void *stream);

/* dK and dV.  Replaces the dK/dV workers of _flash_attn_bwd
 * (original_kernel.py:1339-1525). */
int kd_attn_bwd_dkdv(const kd_attn_args *a, const void *plan, int64_t plan_bytes, void *stream);

/* Whole backward: dQ with Delta (kd_attn_bwd_dq_delta), then dK/dV.  Replaces
 * attention_backward_adapter (original_kernel.py:1806-1898). */
int kd_attn_bwd(const kd_attn_args *a, const void *plan, int64_t plan_bytes, void *stream);

/* The whole backward as kd_attn_bwd, with a->delta ignored: its workspace
 * (2 * B*H*T floats) lives in a library-owned device array of
 * KD_NOALLOC_WORKSPACE_FLOATS floats (16 MiB) on each GPU, held until the
 * process ends, and no call allocates.  No counterpart in the reference: this
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc).  B*H*T above
 * KD_NOALLOC_WORKSPACE_FLOATS / 2 returns KD_ERR_UNSUPPORTED.  Every call on one
 * GPU uses that GPU's one array, so calls that overlap on one GPU (other
 * streams or threads) race and must be ordered by the caller.  The first call
 * on a device resolves the array's address; that call may itself be made
 * inside a HIP graph capture (no warm-up call is needed). */
#define KD_NOALLOC_WORKSPACE_FLOATS (1 << 22)
int kd_attn_bwd_noalloc(const kd_attn_args *a, const void *plan, int64_t plan_bytes, void *stream);

/* The 64-bit masks of every 64x64 tile of a built plan, from the same
 * functions the attention kernels apply to PARTIAL tiles: rows [B, nT, nT, 64]
 * (bit j of entry r: query 64 qt + r may see key 64 kt + j) and cols
 * [B, nT, nT, 64] (bit r of entry j: query 64 qt + r may see key 64 kt + j).
 * An inspection aid (the kernels never store them); no reference counterpart,
 * the reference evaluates original_kernel.py:478-517 per element.  T is at
 * most 65535 * 64 here (KD_ERR_UNSUPPORTED beyond). */
int kd_tile_masks(const void *plan, int64_t plan_bytes, int32_t B, int32_t T, int32_t D, uint64_t *rows,
                  uint64_t *cols, void *stream);

/* Dense bool mask [B, H, T, T] (element strides b, h, q, k) from the plan's
 * codes.  Replaces the RETURN_ATTENTION_MASK store of _flash_attn_fwd
 * (original_kernel.py:519-545). */
int kd_mask_dense(const void *plan, int64_t plan_bytes, int32_t B, int32_t H, int32_t T, int32_t D, uint8_t *out,
                  const int64_t *strides, void *stream);

/* y = x R with R = diag(signs) H_D / sqrt(D) (or x R^T when inverse), per
 * row, in a fixed fp32 evaluation order (bit-reproducible); optionally
 * max |y| per (b, h) into amax.  The reference only names this operation
 * (README.md:68-71, :77: generate_hadamard_signs / hadamard_transform). */
int kd_hadamard(const kd_rot_args *a, void *stream);

/* fp8 e4m3 copy of a rotated Q or K for the fp8 QK^T variant of the
 * attention kernels (kd_attn_args.q8 / k8).  No counterpart in the reference,
 * which has no fp8 path; the operation is specified by the build. */
int kd_quant_fp8(const kd_quant_args *a, void *stream);

/* amax[b H + h] = max |x| over (t, d) of the bf16 / fp16 [B, H, T, D] tensor
 * a->x (a->x_strides; the other fields of a are not read), exact in fp32, for
 * kd_quant_fp8 when no rotation pass (kd_hadamard with amax) produced it.
 * Every element of amax is written; nothing needs to be zeroed first.  No
 * counterpart in the reference, which has no fp8 path. */
int kd_absmax(const kd_quant_args *a, float *amax, void *stream);

/* Cocktail-party head forward: span_lo/hi, mask_pos, h_ctx, h_spans and
 * scores.  Replaces the Python double loop and einsum of GPTModel.forward
 * (model.py:263-298). */
int kd_span_scores(const kd_span_args *a, void *stream);

/* Its backward: dh = d scores / d h times dscores, from the forward's
 * span_lo/hi, mask_pos, h_ctx and h_spans (the autograd of model.py:287-296). */
int kd_span_scores_bwd(const kd_span_args *a, void *stream);

/* sizeof(kd_span_args), for binding checks. */
void kd_struct_sizes4(size_t *span);

#ifdef __cplusplus
}
#endif
#endif /* KDATTN_H */
