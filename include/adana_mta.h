/*
 * adana_mta.h -- C ABI of the MI355X (gfx950) ADana-family optimizer step.
 *
 * One multi-tensor kernel updates every (param, grad, m, v[, tau]) of a
 * parameter list in a single pass over HBM and produces the per-tensor
 * diagnostics the reference stores in the optimizer state.
 *
 * What each entry point replaces in the reference (mlexpos/adana):
 *
 *   adana_step_scalars_init  <- the host scalar code of ADana.step
 *        (src/optim/adana.py:163-208: g2, g3, schedule_factor, alpha, the six
 *        0-d device tensors) and the 0-d tensor arithmetic inside the compiled
 *        update (:104 ``1 - alpha``, :114 ``1.0 + step``, :119 pow, :126
 *        ``(-g3) * gamma_3_factor``, :139-143 weight-decay factor) and
 *        DANA_STAR_MK4.step (src/optim/dana_star_mk4.py:217-272, :154 min_p);
 *        with adana_hparams.foreach, the foreach path's (adana.py:171-176,
 *        :245-262, :316-365; dana_star_mk4.py:455-456).
 *   adana_plan_layout        <- the per-tensor Python loop itself
 *        (src/optim/adana.py:184-216; src/optim/dana_star_mk4.py:243-282):
 *        instead of one compiled call per tensor, tensors are laid end to end
 *        in a virtual index space cut into fixed-size work chunks.
 *   adana_plan_index         <- (same loop) the chunk -> first-tensor index the
 *        kernel uses to find its tensors without a search.
 *   adana_mta_step           <- ADana._update_param_compiled
 *        (src/optim/adana.py:81-153) and DANA_STAR_MK4._update_param_compiled
 *        (src/optim/dana_star_mk4.py:105-205) for ALL tensors of the list,
 *        plus the diagnostics stored at src/optim/adana.py:221-225 /
 *        src/optim/dana_star_mk4.py:290-294; with ADANA_VARIANT_MANAU, the
 *        eager Dana-Star-MK4 branch of Manau.step (src/optim/manau.py:504-613)
 *        for the parameters Manau does not give to Muon; with ADANA_FOREACH,
 *        the use_foreach=True path's _foreach_step_group and
 *        _foreach_compute_kernel_impl (src/optim/adana.py:229-370;
 *        src/optim/dana_star_mk4.py:298-536) for all of a group's tensors.
 *   adana_manau_scalars_init <- that branch's host scalars (manau.py:539-555,
 *        :606-610 and the Python-float operands of its tensor ops).
 *   adana_grad_clip_norm     <- the gradient-norm clipping the training loop
 *        runs before every step (src/optim/base.py:250-257 ->
 *        src/distributed/backend.py:33-35 -> torch.nn.utils.clip_grad_norm_):
 *        total norm and clip coefficient on the device.
 *   adana_mta_step_scaled    <- clip_grad_norm_'s in-place gradient scaling
 *        fused into adana_mta_step's gradient load.
 *   adana_grad_scale         <- the same scaling as a separate in-place pass
 *        (for a gradient list no fused step consumes).
 *   adana_order_stats        <- the tau order statistics of the Dana-Star
 *        state (TauStatsCollector._extract_tau_statistics,
 *        src/optim/tau_stats_collector.py:131-160, which copies every tau
 *        tensor to the host and calls compute_tau_order_statistics, :336-376:
 *        np.sort, then the sorted values at ranks floor(1.1^k) - 1 from both
 *        ends): exact values at given ranks, selected on the GPU.
 *   adana_mta_step_noalloc   <- adana_mta_step with its scratch in a static
 *        device array (no reference counterpart: for callers that cannot
 *        allocate).
 *   adana_last_error, adana_abi_version, adana_workspace_bytes,
 *        adana_order_stats_workspace, adana_order_stats_workspace_compact:
 *        plumbing (no reference counterpart).
 *
 * Ownership: the library allocates nothing (adana_mta_step_noalloc's static
 * scratch is part of the loaded code object); every device buffer is owned by
 * the caller (PyTorch's caching allocator in the Python binding) and only
 * borrowed for the call.  Launches are asynchronous on the caller's HIP
 * stream; nothing synchronises the host, except adana_order_stats (host-driven
 * between its passes).  Errors: functions return 0 on
 * success or a negative code; adana_last_error() returns the message of the
 * calling thread's last failure.
 */
#ifndef ADANA_MTA_H
#define ADANA_MTA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ADANA_ABI_VERSION 8

/* Elements per work chunk (one 256-thread workgroup, one 16-byte vector per
 * thread per array).  Tensors start at multiples of ADANA_ALIGN_ELEMS in the
 * virtual index space, so every vector belongs to exactly one tensor, and a
 * tensor that would cross a chunk boundary from inside a chunk starts at the
 * next boundary (adana_plan_layout). */
#define ADANA_CHUNK_ELEMS 1024
#define ADANA_ALIGN_ELEMS 4
/* Scalar classes (distinct (group, step) pairs) one launch can carry. */
#define ADANA_MAX_CLASSES 8
/* Chunk partials one fold workgroup of the diagnostics combine reduces.
 * Tensors of at most ADANA_DIRECT_CHUNKS chunks get no fold workgroups: the
 * finalize step sums their chunk partials directly; a larger tensor has two
 * folds or more. */
#define ADANA_FOLD_CHUNKS 512
#define ADANA_DIRECT_CHUNKS 512

/* variant_flags of adana_mta_step */
#define ADANA_VARIANT_STAR 0x1u  /* Dana-Star(-MK4): tau state and estimator   */
#define ADANA_GRAD_BF16    0x2u  /* gradients are bfloat16 (else float32)      */
#define ADANA_PARAM_BF16   0x4u  /* param = fp32 master; param_lp = bf16 copy  */
#define ADANA_WRITE_GRAD   0x8u  /* adana_mta_step_scaled: store the scaled
                                    gradient back into grad                   */
#define ADANA_VARIANT_MANAU 0x10u /* Manau's Dana-Star-MK4 branch: tau state,
                                    Manau's op order; float32 only; scalars
                                    from adana_manau_scalars_init            */
#define ADANA_STATE_BF16   0x20u /* the reference's own bfloat16 path: param,
                                    m, v, tau (and, with ADANA_GRAD_BF16,
                                    which it requires, grad) are bfloat16;
                                    d_diag holds 5 bfloat16 per tensor;
                                    excludes ADANA_PARAM_BF16                */
#define ADANA_NUMERICS_EAGER 0x40u /* the update as the reference's ATen ops
                                    run it with torch.compile disabled (lerp_
                                    and addcmul_ as single-rounded FMAs; with
                                    ADANA_STATE_BF16 every op rounded to
                                    bfloat16).  Without it: the reference's
                                    default torch.compile path (Inductor's
                                    forms: products and sums rounded one by
                                    one, binary32 throughout, bfloat16 state
                                    rounded only where it is stored).  The
                                    scalars must come from hparams with the
                                    same choice (adana_hparams.eager).        */
#define ADANA_FOREACH      0x80u /* the reference's use_foreach=True path
                                    (_foreach_compute_kernel_impl,
                                    src/optim/adana.py:310-370,
                                    src/optim/dana_star_mk4.py:395-536): its
                                    op forms (no addcmul, ATen's lerp in both
                                    modes, tau_reg = maximum(p_est, min_p),
                                    mfac = nt * (|m| / tau_reg), p += p * wdf)
                                    and scalars (adana_hparams.foreach), with
                                    either numerics (compiled on bfloat16
                                    state: m and tau rounded to bfloat16 by
                                    ATen's lerp, the rest binary32; eager:
                                    every op rounded); excludes
                                    ADANA_VARIANT_MANAU                       */

/* adana_tensor_desc.flags */
#define ADANA_DESC_VEC_OK  0x1u  /* param, m, v, tau and param_lp aligned for
                                    the vector path: 16 bytes for float32
                                    arrays, 8 for bfloat16 ones (the gradient,
                                    in adana_plan.grad, is checked by the
                                    kernel itself)                            */

/* Error codes */
#define ADANA_OK              0
#define ADANA_E_INVALID     (-1)
#define ADANA_E_HIP         (-2)
#define ADANA_E_UNSUPPORTED (-3)

/* One tensor of the list.  64 bytes; the array lives in device memory.  Its
 * gradient pointer is not here but in adana_plan.grad, a separate array: a
 * training loop brings new gradient tensors every step
 * (zero_grad(set_to_none=True), src/optim/base.py:269-289), and re-pointing
 * them rewrites 8 bytes per tensor instead of a descriptor. */
typedef struct adana_tensor_desc {
    void       *param;     /* float32 param, or the float32 master copy      */
    const void *reserved0; /* unused (0)                                     */
    float      *m;         /* first moment, float32 (bfloat16 with
                              ADANA_STATE_BF16, as are v and tau)            */
    float      *v;         /* second moment                                  */
    float      *tau;       /* Dana-Star tau (NULL otherwise)                 */
    void       *param_lp;  /* bfloat16 param written as RNE(master), or NULL */
    int64_t     numel;
    int32_t     sclass;    /* index into the launch's scalar classes         */
    uint32_t    flags;     /* ADANA_DESC_* bits                              */
} adana_tensor_desc;

/* A laid-out tensor list: host struct holding device pointers (all device
 * arrays are owned by the caller).  Built with adana_plan_layout (host part)
 * and adana_plan_index (chunk_first). */
typedef struct adana_plan {
    const adana_tensor_desc *desc;   /* device, n_tensors entries              */
    const void *const *grad;         /* device, n_tensors gradient pointers:
                                        float32 or bfloat16, numel elements
                                        each, any 2- or 4-byte alignment     */
    const int64_t *vstart;           /* device, n_tensors + 1 (layout output)  */
    const int32_t *chunk_first;      /* device, n_chunks (adana_plan_index)    */
    const int32_t *fold_first;       /* device, n_tensors + 1 (layout output)  */
    int32_t n_tensors;
    int32_t reserved;
    int64_t n_chunks;
    int64_t n_folds;
} adana_plan;

/* Hyper-parameters of one parameter group (reference ctor arguments and
 * group keys, src/optim/adana.py:32-57). */
typedef struct adana_hparams {
    double  peak_lr;        /* the constructor's lr (self.lr)                */
    double  delta;          /* group['delta']                                */
    double  kappa;          /* self.kappa                                    */
    double  epsilon;        /* group['epsilon']                              */
    double  weight_decay;   /* group['weight_decay']                         */
    double  clipsnr;        /* self.clipsnr (ignored unless has_clip)        */
    double  wd_ts;          /* self.wd_ts                                    */
    double  gamma_3_factor; /* self.gamma_3_factor                           */
    int32_t has_clip;       /* self.clipsnr is not None                      */
    int32_t wd_decaying;    /* self.wd_decaying                              */
    int32_t eager;          /* 1: scalars for ADANA_NUMERICS_EAGER launches  */
    int32_t foreach;        /* scalars for ADANA_FOREACH launches: 1 with
                               float32 parameters, 2 with bfloat16 ones (the
                               path's step tensor has the parameters' dtype);
                               0: the per-tensor path                        */
} adana_hparams;

/* Per-step binary32 scalars of one (group, step) class, each computed on the
 * host exactly as the reference's 0-d tensor ops round it.  64 bytes.  The
 * foreach path (adana_hparams.foreach) computes alpha as the binary32
 * quotient fp32(delta) / (fp32(delta) + t), t in the parameters' dtype
 * (src/optim/adana.py:258-259), takes ATen's lerp coefficient from alpha
 * rounded to bfloat16 when the parameters are bfloat16, and uses the three
 * fields marked below with their foreach meaning. */
typedef struct adana_step_scalars {
    float   a;          /* alpha = fp32(delta / (delta + t))                 */
    float   oma;        /* 1 - alpha                                         */
    float   lerp_coef;  /* alpha if |alpha| < 0.5 else alpha - 1 (ATen lerp) */
    float   s;          /* fp32(t)                                           */
    float   eps;        /* fp32(epsilon)                                     */
    float   pw;         /* ADana: (1 + s) ** (1 - kappa), by pow_mode        */
    float   min_p;      /* Dana-Star: 1 / (1 + s)                            */
    float   clip;       /* fp32(clipsnr)                                     */
    float   c3;         /* (-lr) * gamma_3_factor; foreach: gamma_3_factor   */
    float   cg2;        /* -lr; foreach: lr                                  */
    float   opw;        /* 1 + weight-decay factor; foreach: the factor wdf
                           of p + p * wdf (adana.py:357-368)                 */
    float   star_exp;   /* fp32(1 - kappa), exponent of Dana-Star's pow      */
    int32_t pow_mode;   /* pow specialisation of 1 - kappa (ADANA_POW_*)     */
    int32_t has_clip;
    int32_t lerp_small; /* |alpha| < 0.5                                     */
    int32_t pow_int;    /* ADANA_POW_INT: the integer exponent               */
} adana_step_scalars;

/* Specialisations of x ** e chosen on the binary64 exponent e.
 * Eager (ATen's pow(Tensor, Scalar)): ONE (e = 0: 1), IDENTITY (e = 1: a
 * copy), SQRT (0.5), RSQRT (-0.5: 1 / sqrt), RECIP (-1), SQUARE (2), CUBE
 * (3), INVSQ (-2: 1 / (x * x)); any other e GENERAL.
 * Compiled (Inductor's pow lowering): ONE (e = 0), IDENTITY (e = 1), SQRT
 * (0.5), INT (any other integer e with |e| < 32: left-to-right binary
 * powering of x, or of 1 / x for e < 0, exponent in pow_int); any other e,
 * -0.5 included, GENERAL.  GENERAL is pow with the exponent rounded to
 * binary32 (ADana's eager scalar: pow in binary64 with the binary64
 * exponent). */
enum {
    ADANA_POW_GENERAL = 0, ADANA_POW_ONE, ADANA_POW_SQRT, ADANA_POW_RSQRT,
    ADANA_POW_RECIP, ADANA_POW_SQUARE, ADANA_POW_CUBE, ADANA_POW_INVSQ,
    ADANA_POW_IDENTITY, ADANA_POW_INT
};

/* Hyper-parameters of one Manau parameter group that its Dana-Star-MK4
 * branch reads (group keys, src/optim/manau.py:121-173, :509-519). */
typedef struct adana_manau_hparams {
    double  delta;
    double  kappa;
    double  mk4A;
    double  mk4B;
    double  clipsnr;
    double  epsilon;
    double  weight_decay;
    double  wd_ts;
    int32_t wd_decaying;
    int32_t reserved;
} adana_manau_hparams;

/* Per-step binary32 scalars of one class of Manau's branch.  Same size as
 * adana_step_scalars: launches with ADANA_VARIANT_MANAU pass an array of
 * these where adana_mta_step takes h_scalars. */
typedef struct adana_manau_scalars {
    float   a;          /* fp32(alpha), alpha the branch's binary64 value    */
    float   oma;        /* fp32(1 - alpha), difference in binary64           */
    float   s;          /* fp32(step) (a weighted step count with weight_time)*/
    float   eps;        /* fp32(epsilon)                                     */
    float   min_p;      /* fp32(1 / (1 + step)), binary64 quotient           */
    float   clip;       /* fp32(clipsnr)                                     */
    float   lr;         /* fp32(lr)                                          */
    float   wdf;        /* fp32(1 - wd / (1 + step / wd_ts) * lr) or
                           fp32(1 - wd * lr), binary64 arithmetic            */
    float   e[3];       /* exponents 1 - kappa, 2 mk4B + 1, 2 (-mk4A - mk4B),
                           rounded to binary32                               */
    int32_t mode[3];    /* ADANA_POW_* of each exponent (binary64 value)     */
    int32_t has_wd;     /* weight_decay != 0                                 */
    int32_t reserved;
} adana_manau_scalars;

int adana_abi_version(void);

/* Copies the calling thread's last error message (NUL-terminated). */
size_t adana_last_error(char *buf, size_t len);

/* Host only.  Scalars of one tensor update at learning rate ``lr``
 * (group['lr']) and per-tensor step ``step`` (state['step'] after += 1). */
int adana_step_scalars_init(adana_step_scalars *out, const adana_hparams *hp,
                            double lr, int64_t step);

/* Host only.  Scalars of one tensor update of Manau's branch at learning
 * rate ``lr`` with the branch's ``step`` (state['step'], or the group's
 * weighted step count when weight_time) and ``alpha`` (manau.py:548-555). */
int adana_manau_scalars_init(adana_manau_scalars *out, const adana_manau_hparams *hp,
                             double lr, double step, double alpha);

/* Host only.  Lays n tensors end to end: writes vstart[0..n] (virtual start
 * of each tensor: the end of the previous one rounded up to a multiple of
 * ADANA_ALIGN_ELEMS, or further up to the next multiple of ADANA_CHUNK_ELEMS
 * when the tensor would otherwise cross that chunk boundary; vstart[n] is the
 * padded total) and fold_first[0..n] (first fold workgroup of each tensor's
 * diagnostics combine: ceil(chunks / ADANA_FOLD_CHUNKS) for a tensor of more
 * than ADANA_DIRECT_CHUNKS chunks, none otherwise; fold_first[n] = *n_folds),
 * and returns the number of
 * work chunks (>= 0), or a negative error code. */
int64_t adana_plan_layout(const int64_t *numel, int32_t n, int64_t *vstart,
                          int32_t *fold_first, int64_t *n_folds);

/* Device.  Fills d_chunk_first[c] (c < n_chunks) with the index of the first
 * tensor whose virtual range reaches chunk c, from the device copy of vstart.
 * Asynchronous on ``stream``; run once per layout. */
int adana_plan_index(const int64_t *d_vstart, int32_t n_tensors, int64_t n_chunks,
                     int32_t *d_chunk_first, void *stream);

/* Bytes of device workspace adana_mta_step needs for ``plan``. */
size_t adana_workspace_bytes(const adana_plan *plan);

/* Device step over one tensor list.
 *   plan        the laid-out list (host struct, device arrays)
 *   h_scalars   host array of n_classes scalar classes (passed by value to
 *               the kernel; no host-to-device copy)
 *   d_workspace device scratch of at least adana_workspace_bytes(plan) bytes
 *               (per-chunk partial sums, their folds, one arrival counter
 *               per tensor, and 32 KB for the pow table a bfloat16-state
 *               Dana-Star launch fills first; contents on entry are ignored)
 *   d_diag      device float[5 * n_tensors]: per tensor current_alpha,
 *               gradient_norm, auto_factor_mean, current_kappa_factor,
 *               m_norm (src/optim/adana.py:221-225); with ADANA_STATE_BF16
 *               5 * n_tensors bfloat16 values instead
 *   stream      hipStream_t (NULL = default stream)
 * All tensors of one call share variant_flags. */
int adana_mta_step(const adana_plan *plan, const adana_step_scalars *h_scalars,
                   int32_t n_classes, uint32_t variant_flags, void *d_workspace,
                   size_t workspace_bytes, float *d_diag, void *stream);

/* Device.  adana_mta_step on clipped gradients: each gradient element is
 * replaced by g * (*d_grad_scale) as it is loaded (rounded to bfloat16 for
 * bfloat16 gradients), which is what torch.nn.utils.clip_grad_norm_'s
 * ``torch._foreach_mul_(grads, clip_coef_clamped)`` leaves in the gradient
 * (torch/nn/utils/clip_grad.py, _clip_grads_with_norm_), so the update and
 * the diagnostics see exactly the clipped gradient.  With ADANA_WRITE_GRAD in
 * variant_flags the scaled gradient is also stored back, leaving grad as the
 * reference's in-place clipping does; without it grad is not modified.
 * d_grad_scale: device float, typically d_clip + 1 of adana_grad_clip_norm. */
int adana_mta_step_scaled(const adana_plan *plan, const adana_step_scalars *h_scalars,
                          int32_t n_classes, uint32_t variant_flags,
                          const float *d_grad_scale, void *d_workspace,
                          size_t workspace_bytes, float *d_diag, void *stream);

/* Bytes of the library's static device scratch behind adana_mta_step_noalloc
 * (per GPU, held until the process ends): room for lists of up to about
 * 4.1 million work chunks (4.2e9 elements), since the step needs 16 bytes per
 * (chunk, tensor) slot, 32 per fold and 4 per tensor. */
#define ADANA_NOALLOC_SCRATCH_BYTES (64u << 20)

/* Device.  adana_mta_step without a workspace argument: the chunk partials
 * and folds go to a static device array of ADANA_NOALLOC_SCRATCH_BYTES, so
 * the call allocates nothing (no hipMalloc, no allocating library call).  No
 * counterpart in the reference: it is for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Returns ADANA_E_UNSUPPORTED, with a message, for a list whose
 * adana_workspace_bytes exceeds ADANA_NOALLOC_SCRATCH_BYTES.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (several
 * streams or threads) race and must be serialised by the caller.  The
 * array's address on each device is looked up on the first call with that
 * device current. */
int adana_mta_step_noalloc(const adana_plan *plan, const adana_step_scalars *h_scalars,
                           int32_t n_classes, uint32_t variant_flags, float *d_diag, void *stream);

/* Device.  The norm half of torch.nn.utils.clip_grad_norm_(params, max_norm)
 * with norm_type 2 (src/optim/base.py:250-257, src/distributed/backend.py:
 * 33-35), over the gradients of ``plan`` (only desc[i].grad, numel and flags
 * are read; grad_flags: 0 for float32 or ADANA_GRAD_BF16 for bfloat16
 * gradients, shared by the whole list).  Writes, in torch's order and dtype
 * (each value rounded to the gradient dtype):
 *   d_norms[i]  ||grad_i||_2 (torch._foreach_norm), or d_norms == NULL
 *   d_clip[0]   total norm = ||(norm_0, ..., norm_{n-1})||_2
 *   d_clip[1]   min(reciprocal(total + 1e-6) * max_norm, 1)  (NaN propagates)
 * Sums of squares are accumulated in binary64.  d_workspace: at least
 * adana_workspace_bytes(plan) bytes (its own, or one not in use by a step
 * running concurrently).  Asynchronous on ``stream``. */
int adana_grad_clip_norm(const adana_plan *plan, uint32_t grad_flags, double max_norm,
                         void *d_workspace, size_t workspace_bytes, float *d_norms,
                         float *d_clip, void *stream);

/* Device.  In place grad_i *= *d_scale for every gradient of ``plan``
 * (clip_grad_norm_'s torch._foreach_mul_; bfloat16 products rounded to
 * bfloat16).  Asynchronous on ``stream``. */
int adana_grad_scale(const adana_plan *plan, uint32_t grad_flags, const float *d_scale,
                     void *stream);

/* Bytes of device workspace adana_order_stats needs. */
size_t adana_order_stats_workspace(int32_t n_tensors, int64_t total_ranks);

/* Bytes of device workspace with which adana_order_stats also compacts: once
 * at most 1/16 of a tensor's values still share a prefix with its wanted
 * ranks, one pass keeps those values (per 65,536-element tile, up to 32 of
 * each thread's 256) and the later passes read only them.  About 1/8 of the
 * wanted tensors' bytes more than adana_order_stats_workspace.  Same
 * arguments as adana_order_stats (h_numel[n_tensors], h_rank_first[n_tensors
 * + 1]); 0 for invalid ones. */
size_t adana_order_stats_workspace_compact(const int64_t *h_numel, const int64_t *h_rank_first,
                                           int32_t n_tensors);

/* Host-driven, synchronous.  Exact order statistics of float32 tensors: for
 * each tensor i (h_tensors[i]: device pointer, h_numel[i] elements, any
 * alignment), the values at ranks h_ranks[h_rank_first[i] ..
 * h_rank_first[i+1]) (0 <= rank < h_numel[i]) of its ascending order as
 * np.sort orders it (NaN last; -0 and +0 equal as values), written to the
 * host array h_values at the same positions.  A multi-rank radix select: 4
 * to 8 passes that each read the tensors once and histogram the next key
 * digit per wanted prefix in LDS; after each pass every rank is narrowed to
 * its next digit on the device, and the host reads back the new prefixes to
 * set up the next pass.  Synchronises ``stream``.  d_workspace: at least
 * adana_order_stats_workspace(n_tensors, h_rank_first[n_tensors]) bytes;
 * with adana_order_stats_workspace_compact(...) bytes or more, the late passes
 * read only the values that can still match (same results).
 * Ranks may come in any order and repeat; ascending ranks save a host sort
 * per pass.  Returns ADANA_E_UNSUPPORTED for a tensor of 2^32 elements or
 * more, or one whose ranks hold more than 4,096 distinct values at some
 * pass (its histograms would not fit in LDS). */
int adana_order_stats(const float *const *h_tensors, const int64_t *h_numel, int32_t n_tensors,
                      const int64_t *h_ranks, const int64_t *h_rank_first, float *h_values,
                      void *d_workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* ADANA_MTA_H */
