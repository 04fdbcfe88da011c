/*
 * C ABI of libapexw_hip.so: the fused ApexW optimizer step and Muon
 * Newton-Schulz kernels for AMD Instinct MI355X (gfx950).
 *
 * Everything is passed as plain pointers and sizes.  Device pointers point into
 * memory owned by the caller (PyTorch tensors); the library never allocates
 * caller-visible memory.  Every entry point validates its arguments before the
 * first write and returns an apexw_status; APEXW_OK means the work was enqueued
 * on `stream` (asynchronous, like a kernel launch).
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   apexw_compact_step   <- pybind step_fused / fused_multi_tensor_adamw_cuda_step
 *                           (apexw/csrc/apexw_cuda.cpp:109-234, :455-513;
 *                           Python wrappers apexw/cuda_extension.py:123-158, :197-215)
 *                           and the Triton bucket launch triton_multi_tensor_adamw_step
 *                           (apexw/triton_kernel.py:2524-2874)
 *   apexw_q8_step        <- pybind step_fused_8bit (apexw/csrc/apexw_cuda.cpp:310-453;
 *                           wrapper apexw/cuda_extension.py:161-194) and
 *                           _adamw_kernel_triton_8bit_batched (apexw/triton_kernel.py:1138-1531)
 *   apexw_grad_clip_coef <- the global-norm clip of _prepare_grads
 *                           (apexw/optimizer.py:242-256: _foreach_norm + vector_norm)
 *   apexw_grad_prepare   <- sanitize / AMP unscale / grad centralization of
 *                           _prepare_grads (apexw/optimizer.py:204-240)
 *   apexw_gemm_nt_bf16   <- the bf16 GEMMs of Newton-Schulz: X @ X.T and the two
 *                           torch.addmm / baddbmm calls (apexw/muon.py:102-108, :187-211)
 *   apexw_gemm_nt_grouped <- the same GEMMs for every Muon matrix of a step in one
 *                           launch (per-shape loop of apexw/muon.py:593-615)
 *   apexw_muon_prepare   <- ApexMuon momentum update and the work-matrix cast /
 *                           normalisation / transpose (apexw/muon.py:763-792, :163-175, :190-200)
 *   apexw_muon_apply     <- the decoupled decay and scaled update of ApexMuon
 *                           (apexw/muon.py:852-858, :752-759)
 *   apexw_muon_coordwise <- ApexMuon._step_single's coordinate-wise fallback for
 *                           vectors and dimensions under 16 (apexw/muon.py:775-799, :841-858)
 *   apexw_state_decode / apexw_state_encode: no counterpart (the reference keeps
 *                           a checkpoint's saved layout, apexw/optimizer.py:2487-2572);
 *                           they convert a state between precision modes on load
 */
#ifndef APEXW_HIP_H
#define APEXW_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define APEXW_ABI_VERSION 24

/* status codes */
enum apexw_status {
  APEXW_OK = 0,
  APEXW_ERR_ARG = 1,      /* invalid argument (null pointer, bad size, bad flag) */
  APEXW_ERR_DTYPE = 2,    /* unsupported dtype combination */
  APEXW_ERR_LAUNCH = 3,   /* the HIP runtime rejected the launch */
  APEXW_ERR_ALIGN = 4,    /* pointer alignment the kernel requires is not met */
  APEXW_ERR_SIZE = 5      /* the work exceeds a fixed-size workspace (allocation-free entry points) */
};

/* element dtype codes */
enum apexw_dtype { APEXW_F32 = 0, APEXW_BF16 = 1, APEXW_F16 = 2, APEXW_U8 = 3, APEXW_I8 = 4 };

/* apexw_tensor.flags: dtype fields (2 bits each) and per-tensor mode bits */
#define APEXW_FLAG_PDT_SHIFT 0          /* param dtype */
#define APEXW_FLAG_GDT_SHIFT 2          /* grad dtype */
#define APEXW_FLAG_MDT_SHIFT 4          /* compact: first-moment dtype */
#define APEXW_FLAG_VDT_SHIFT 6          /* compact: second-moment dtype */
#define APEXW_FLAG_QUAD (1u << 8)       /* one v per 4 consecutive elements */
#define APEXW_FLAG_WD (1u << 9)         /* apply decoupled weight decay */
#define APEXW_FLAG_NF4 (1u << 10)       /* 8-bit: NF4 packed m (else INT8 m) */
#define APEXW_FLAG_GENERIC (1u << 11)   /* 8-bit: per-parameter ("generic") rounding order */
#define APEXW_FLAG_DENSE (1u << 12)     /* 8-bit / ultra step: dense m and v (bf16 or fp32; MDT / VDT
                                           fields), element-wise update in units of 2048 elements:
                                           8-bit tensors under 64 elements, small ultra tensors */
#define APEXW_FLAG_SCALAR (1u << 13)    /* pointers not 16-byte aligned: element-wise path */
#define APEXW_FLAG_FACTORED (1u << 14)  /* factored second moment: stepped by apexw_factored_step;
                                           the compact and 8-bit step kernels skip the row */
#define APEXW_FLAG_M6 (1u << 15)        /* factored 8-bit: packed 6-bit m (4 codes in 3 bytes) */
#define APEXW_FLAG_GC (1u << 16)        /* step kernels and clip: grad centralization folded in; the grad
                                           is read raw and g - mean(row) taken in its dtype (after
                                           sanitize / unscale, before the clip).  The fp32 row means
                                           (apexw_grad_row_means) and the row length: in compact
                                           tables m_scale and block; in 8-bit / ultra tables (whose
                                           m_scale and block hold the quantization scales and block)
                                           the descriptor's apexw_row_means entry (hparams.rows, and
                                           the clip's rows argument) */
#define APEXW_FLAG_VSCALE (1u << 18)    /* compact step: v holds the second moment times a dynamic scale
                                           (fp16 v): v_scale points at {scale_v, sqrt(scale_v)} (fp32,
                                           scale a power of two), read by the cold and replay modes */
#define APEXW_FLAG_ULTRA (1u << 17)     /* 8-bit step kernel, precision "ultra": INT8 m with one scale per
                                           block (m_scale), dense v (VDT field), no v scales */

/*
 * One tensor of a multi-tensor launch (device-resident array, 64 bytes each).
 * compact: m/v are the moment tensors (dtypes in flags), scales unused, block = 0.
 * 8-bit:   m is the NF4 (uint8, 2 per byte, even element in the high nibble) or
 *          INT8 code buffer, v the log-uint8 codes (n/4 entries when QUAD),
 *          m_scale / v_scale the fp32 per-block scales, block the block size.
 * factored (APEXW_FLAG_FACTORED): v is the fp32 row EMA (rows entries) and
 *          v_scale the fp32 column EMA (cols entries); m is INT8 codes, packed
 *          6-bit codes (APEXW_FLAG_M6) or, with block = 0, a 16-bit tensor of the
 *          MDT dtype; m_scale the per-block scales of quantized m.
 */
typedef struct apexw_tensor {
  void* p;
  const void* g;
  void* m;
  void* v;
  float* m_scale;
  float* v_scale;
  int64_t n;
  uint32_t flags;
  uint32_t block;
} apexw_tensor;

/*
 * Work-unit (chunk) table entry: unit `unit` of tensor `tensor`.  A unit is
 * APEXW_COMPACT_UNIT consecutive elements in compact mode and one quantization
 * block in 8-bit mode.  Units of one tensor must be contiguous in the table.
 */
typedef struct apexw_unit {
  uint32_t tensor;
  uint32_t unit;
} apexw_unit;

#define APEXW_COMPACT_UNIT 2048

/* apexw_hparams.mode */
#define APEXW_MODE_COLD 0     /* first step of a plan: _multi_tensor_step rounding */
#define APEXW_MODE_REPLAY 1   /* FastExecutionPlan.execute_foreach rounding */
#define APEXW_MODE_NATIVE 2   /* torch._fused_adamw_ rounding (homogeneous 16-bit groups) */
#define APEXW_MODE_SINGLE 3   /* the per-parameter in-backward update of enable_fused_backward
                                 (ApexW._step_single_param_fused, apexw/optimizer.py:2373-2471):
                                 fp32 m = b1 m + (1-b1) g, lookahead b1 m + (1-b1) g with the new m,
                                 denominator sqrt(v) + eps_scaled (no floor), p decayed then
                                 p + (-step_size * num) / den; INT8 m requantised without the
                                 scale EMA and without SR; compact: full-size m and v only.
                                 Grads are used as given (no sanitize, clip or AMP flags). */

/* apexw_hparams.flags */
#define APEXW_HP_SR (1u << 0)         /* stochastic rounding of 16-bit params / codes */
#define APEXW_HP_SR_V (1u << 1)       /* compact: SR of the 16-bit v EMA (beta2 >= 0.995 and SR) */
#define APEXW_HP_SANITIZE (1u << 2)   /* NaN -> 0, +-Inf -> +-65504 on the grads */
#define APEXW_HP_CLIP (1u << 3)       /* multiply grads by *clip_coef (rounded to grad dtype) */
#define APEXW_HP_LERP_HI (1u << 4)    /* m lerp weight (1 - beta1) >= 0.5: end-based form */
#define APEXW_HP_LOOK_HI (1u << 5)    /* 8-bit lookahead lerp weight (beta1) >= 0.5 */
#define APEXW_HP_UNSCALE (1u << 6)    /* AMP: grads times grad_inv_scale (after sanitizing): in the
                                         grad dtype for compact and before a clip, in fp32 after
                                         the step's nan_to_num otherwise (8-bit, factored) */
#define APEXW_HP_FV_SANITIZE (1u << 7) /* factored: nan_to_num(0, +-65504) on the fp32 grad */
#define APEXW_HP_AMP (1u << 8)         /* a GradScaler step read on the device: the kernels take
                                          step_size, eps_scaled, bc2_sqrt and grad_inv_scale from
                                          *amp (apexw_amp_prepare) and return before any write when
                                          amp->skip (found_inf); APEXW_HP_UNSCALE is set with it */
#define APEXW_HP_NESTEROV (1u << 9)    /* nesterov=True.  8-bit / ultra steps: the dense and ultra
                                          rows' numerator is lerp(g, m, beta1) instead of m (the NF4 /
                                          INT8 blocks take Nesterov through gain_hi = gain_lo = 1).
                                          Compact step (cold and replay modes, no APEXW_HP_AMP): quad
                                          tensors take lerp(g, m, beta1) (look_coef, APEXW_HP_LOOK_HI),
                                          the others p += gain_hi * m / d, then p += gain_lo * g / d,
                                          each rounded to p's dtype, never stochastic (gain_hi =
                                          -step_size * beta1, gain_lo = -step_size * (1 - beta1)) */
#define APEXW_HP_CAUTIOUS (1u << 10)   /* cautious=True.  Compact step: see
                                          apexw_compact_cautious_count.  8-bit / ultra steps: the numerator is
                                          m' x q_t where m' g >= 0, else 0 (q_t = 1 / max(c_t / n_t,
                                          1e-3), c_t = hparams.counts[t] written by
                                          apexw_q8_cautious_count); the blocks take it with
                                          look_coef = 0 under APEXW_HP_LOOK_HI (numerator m', no
                                          lookahead) and gain_lo = 0 */
#define APEXW_HP_AMSGRAD (1u << 11)    /* amsgrad=True.  Compact step (cold, replay and native modes;
                                          full-size v only, quad descriptors ignore it): the
                                          denominator takes vmax = max(max_v[t], v') instead of v'
                                          and vmax is stored back to max_v[t] (VDT dtype, n elements,
                                          16-byte aligned unless APEXW_FLAG_SCALAR).  Cold and replay:
                                          v' as stored; native: the fp32 v' (torch._fused_adamw_),
                                          vmax stored rounded.  A NaN on either side gives NaN. */
#define APEXW_HP_LION (1u << 12)       /* lion=True.  Compact step (cold and replay modes; no
                                          APEXW_HP_NESTEROV / _CAUTIOUS / _AMSGRAD, no quad rows): with
                                          g' the prepared grad in m's dtype, p += a * sign(lerp(g', m,
                                          beta1)) (look_coef / APEXW_HP_LOOK_HI; the lerp rounded to m's
                                          dtype, sign(0) = sign(NaN) = 0), a = -gain_hi (gain_hi = lr),
                                          rounded to p's dtype when p and m share a 16-bit dtype; then
                                          m = lerp(m, g', 1 - beta2) (lerp_coef / APEXW_HP_LERP_HI).  v
                                          is neither read nor written (descriptors may point v at m). */
#define APEXW_HP_SLOW (1u << 13)       /* beta3 (AdEMAMix).  Compact step (cold and replay modes; no
                                          APEXW_HP_CAUTIOUS / _LION / _AMP, no quad rows): a slow first
                                          moment s = slow[t] (m's dtype, n elements, 16-byte aligned
                                          unless APEXW_FLAG_SCALAR) follows m's update with beta3 (the
                                          replay's lerp when the grad and m dtypes match, else mul by
                                          beta3 rounded to m's dtype then add (1 - beta3) g; fp32 m:
                                          lerp), lerp3_coef / APEXW_HP_LERP3_HI the lerp's coefficient
                                          as lerp_coef's; the numerator is m + slow_ratio s (fp32 in
                                          the cold mode for an fp32 p over 16-bit m, else in m's dtype:
                                          for a 16-bit m with r = slow_ratio rounded to it, fma(r, s, m)
                                          rounded, but m + rnd(r s) rounded in each tensor's last n % 32
                                          elements, as torch's CPU add with alpha), then one
                                          round-to-nearest addcdiv into p (nesterov ignored). */
#define APEXW_HP_LERP3_HI (1u << 14)   /* APEXW_HP_SLOW: the slow lerp weight (1 - beta3) >= 0.5 */
#define APEXW_HP_GRAD_DTYPES (1u << 15) /* compact step (cold and replay modes) and its cautious count: some
                                          descriptor's grad dtype (GDT) differs from its parameter's
                                          (torch's Tensor.grad_dtype); such descriptors are stepped only
                                          when this flag is set and skipped otherwise.  The grads are
                                          prepared in their own dtype and read as fp32 values, as the
                                          reference's foreach order does. */

/* Step scalars of one launch, written on the device by apexw_amp_prepare (32 bytes). */
typedef struct apexw_amp_dyn {
  float step_size, eps_scaled, bc2_sqrt, grad_inv_scale;
  uint32_t skip;         /* GradScaler found an inf / NaN: no update this step */
  uint32_t reserved[3];
} apexw_amp_dyn;

/* Grad centralization's row means of descriptor i of an 8-bit / ultra table
 * (APEXW_FLAG_GC): means[r] is the fp32 mean of row r, rows of row_len
 * elements (written by apexw_grad_row_means; 16 bytes). */
typedef struct apexw_row_means {
  const float* means;
  int64_t row_len;
} apexw_row_means;

/* Host-computed step scalars (the reference computes them in double). */
typedef struct apexw_hparams {
  float beta1, one_minus_beta1, beta2, one_minus_beta2;
  float wd_factor;      /* compact: 1 - lr*wd; 8-bit: max(1 - lr*wd, 0) */
  float step_size;      /* lr*sqrt(1-beta2^t)/(1-beta1^t); native mode: lr/(1-beta1^t) */
  float eps_scaled;     /* eps*sqrt(1-beta2^t) */
  float eps;            /* 8-bit: denominator floor; native mode: eps */
  float lerp_coef;      /* m lerp toward g: w if w < 0.5 else w - 1 (w = fp32(1 - beta1)) */
  float look_coef;      /* 8-bit lookahead lerp(g, m, beta1): same rule with w = fp32(beta1) */
  float bc2_sqrt;       /* native mode: sqrt(1-beta2^t) */
  float gain_hi, gain_lo;   /* 8-bit "Nesterov-SNR" gains 1+0.2*beta1, 1-0.35*beta1; compact
                               with APEXW_HP_NESTEROV: the two addcdiv scalars (see the flag) */
  const float* clip_coef;   /* device scalar written by apexw_grad_clip_coef, or NULL */
  uint64_t seed;
  uint32_t step;
  uint32_t mode;
  uint32_t flags;
  float grad_inv_scale; /* with APEXW_HP_UNSCALE: 1 / AMP grad scale (GradScaler); negated for
                           maximize=True (the grads are negated too; finite, non-zero) */
  const apexw_amp_dyn* amp;  /* with APEXW_HP_AMP: this launch's device-side step scalars */
  const apexw_row_means* rows;  /* 8-bit / ultra tables with APEXW_FLAG_GC rows: one entry per
                                   descriptor of the table, else NULL */
  unsigned long long* counts;   /* APEXW_HP_CAUTIOUS: one counter per descriptor of the table */
  void* const* max_v;           /* APEXW_HP_AMSGRAD: one device pointer per descriptor of the table
                                   (the running max of v), in device memory, else NULL */
  float beta3, one_minus_beta3; /* APEXW_HP_SLOW: the slow moment's EMA factors */
  float lerp3_coef;             /* APEXW_HP_SLOW: its lerp coefficient (lerp_coef's rule, w = fp32(1 - beta3)) */
  float slow_ratio;             /* APEXW_HP_SLOW: alpha (1 - beta1^t) / (1 - beta3^t) */
  void* const* slow;            /* APEXW_HP_SLOW: one device pointer per descriptor (exp_avg_slow), else NULL */
} apexw_hparams;          /* 144 bytes */

/*
 * GradScaler hands the optimizer its scale and found_inf as device tensors
 * (torch's _step_supports_amp_scaling protocol); the reference reads both on
 * the host (found_inf.item(), apexw/optimizer.py:3465-3467; grad_scale
 * reciprocal, :5530-5537), which waits for the backward to finish.  This call
 * reads them on the device instead, for up to APEXW_AMP_MAX_LAUNCHES launches
 * of one step:
 *   skip  = (*found_inf != 0)
 *   s     = *skips  (steps skipped so far on the device); when skip, *skips = s + 1
 *   t     = launch.step - (s - skips_folded)   (the host's step count, which counted
 *           every step, less the skips it has not subtracted yet)
 *   bc1   = 1 - beta1^t, bc2 = 1 - beta2^t (double)
 *   kind 0: step_size = lr sqrt(bc2) / bc1, eps_scaled = eps sqrt(bc2)
 *   kind 1 (torch._fused_adamw_ order): step_size = lr / bc1, bc2_sqrt = sqrt(bc2)
 *   grad_inv_scale = 1 / *grad_scale (fp32)
 * into dyn[i].  launches: HOST array (copied into the launch); skips: one device
 * int32, zero at first use, owned by the caller's plan.
 */
#define APEXW_AMP_MAX_LAUNCHES 16
typedef struct apexw_amp_launch {
  double lr, beta1, beta2, eps;
  double step;           /* the host's (already advanced) step count for this launch */
  uint32_t kind;         /* 0 or 1, as above */
  uint32_t reserved;
} apexw_amp_launch;      /* 48 bytes */
int apexw_amp_prepare(const float* found_inf, const float* grad_scale, int32_t* skips, int32_t skips_folded,
                      const apexw_amp_launch* launches, int32_t n_launches, apexw_amp_dyn* dyn, void* stream);

/* ABI version of the loaded library (APEXW_ABI_VERSION). */
int apexw_abi_version(void);

/*
 * Validate one tensor descriptor (HOST copy) before it is uploaded into a
 * device table: kind 0 = compact step, 1 = 8-bit step, 2 = 8-bit step on the
 * full-block kernel (bf16 or fp32 params, NF4 m, quad v, 2048-element blocks),
 * 3 = compact step in APEXW_MODE_SINGLE (full-size v only), 4 = factored
 * tensor (APEXW_FLAG_FACTORED row of either table), 5 = row of the ultra step
 * (APEXW_FLAG_ULTRA or APEXW_FLAG_DENSE; kind 1 refuses ultra rows).  Checks the dtype
 * combination, block size and the 16-byte alignment the vector path needs
 * (unless APEXW_FLAG_SCALAR is set).  Mirrors the per-call tensor checks of the
 * reference's pybind glue (apexw/csrc/apexw_cuda.cpp:109-180, :310-380), done
 * once per execution plan instead of per step.
 */
int apexw_check_tensor(const apexw_tensor* t, int32_t kind);

/*
 * The scalar argument checks that a step entry point applies before it enqueues
 * anything, without enqueueing: kind APEXW_LAUNCH_COMPACT (apexw_compact_step),
 * APEXW_LAUNCH_Q8 (apexw_q8_step), APEXW_LAUNCH_ULTRA (apexw_ultra_step) or
 * APEXW_LAUNCH_FACTORED (apexw_factored_step; n_fast counts 0) or APEXW_LAUNCH_CAUTIOUS
 * (apexw_q8_cautious_count / apexw_compact_cautious_count; n_fast counts 0).  The entry points
 * run exactly these checks, so a caller that checks every launch of a step first
 * can refuse the whole step before any parameter changes.  Replaces the
 * reference's validate-before-mutate order around step_fused_8bit
 * (_execute_cuda_8bit_partition, apexw/optimizer.py:3184-3356) and its step
 * counter rollback on a refused launch (:3806, :3888, :3969).
 */
#define APEXW_LAUNCH_COMPACT 0
#define APEXW_LAUNCH_Q8 1
#define APEXW_LAUNCH_FACTORED 4
#define APEXW_LAUNCH_ULTRA 5
#define APEXW_LAUNCH_CAUTIOUS 6   /* apexw_q8_cautious_count, apexw_compact_cautious_count */
int apexw_check_launch(int32_t kind, int32_t n_tensors, int64_t n_units, int64_t n_fast_units,
                       int64_t n_fast_f32_units, const apexw_hparams* hp);

/*
 * The cautious mask's counts of one 8-bit / ultra step (cautious=True,
 * apexw/optimizer.py:4585-4588, :4672-4675, :4726-4729): sets hp->counts[t] to
 * the number of elements of descriptor t whose updated first moment
 * m' = lerp(m, g', 1 - beta1) (g' the grad as the step prepares it) has
 * m' g' >= 0, over the units given (all of the step's units).  hp as for the
 * step that follows (its mode, flags and scalars; APEXW_HP_CAUTIOUS and counts
 * set).  The step reads the counts in the same stream order.  No counterpart
 * kernel in the reference, which forms the mask on the host.
 */
int apexw_q8_cautious_count(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units, int64_t n_units,
                            const apexw_hparams* hp, void* stream);

/*
 * The same counts for a compact-precision step (compact, full and auto; cautious=True,
 * apexw/optimizer.py:5728-5731, :5847-5864, :1272-1275, :1321-1328): elements whose
 * updated first moment m' and prepared grad g' have m' g' >= 0, the product formed
 * in fp32 (quad v and the cold mode) or, in the replay mode, in the grad dtype after
 * m' is cast to it.  The step (APEXW_HP_CAUTIOUS) turns each count into
 * 1 / max(mean, 1e-3), in fp32 for quad v and in the parameter's dtype otherwise.
 */
int apexw_compact_cautious_count(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units,
                                 int64_t n_units, const apexw_hparams* hp, void* stream);

/*
 * Compact-precision fused AdamW step over every tensor of the table in one
 * launch.  p, m, v are updated in place, g is read only.
 */
int apexw_compact_step(const apexw_tensor* tensors, int32_t n_tensors,
                       const apexw_unit* units, int64_t n_units,
                       const apexw_hparams* hp, void* stream);

/*
 * The "ultra" precision's step (ApexW._step_ultra, apexw/optimizer.py:4640-4686
 * for its INT8-m tensors, :4688-4735 for its small fp32-moment tensors): units of
 * rows flagged APEXW_FLAG_ULTRA (one INT8-m block each; dense v, no v scales)
 * or APEXW_FLAG_DENSE (2048 elements each), validated with apexw_check_tensor
 * kind 5.  Cold and replay modes round alike here (the reference's replay calls
 * the same function).  Replaces the general 8-bit launch for these rows, whose
 * kernel would hold them at a lower occupancy.
 */
int apexw_ultra_step(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units, int64_t n_units,
                     const apexw_hparams* hp, void* stream);

/*
 * 8-bit fused step: dequantize m (NF4 or INT8) and v (log-uint8) with their
 * block scales, AdamW with the SNR lookahead gain, write p, requantize m and v
 * with block absmax / max scales (EMA-max 0.9 / 0.95).  One unit = one block.
 * Units are laid out in three ranges: units[0, n_fast_units) belong to bf16
 * tensors accepted by apexw_check_tensor(t, 2) and run on the full-block
 * kernel; the next n_fast_f32_units belong to fp32 tensors accepted by
 * apexw_check_tensor(t, 2) and run on its fp32 variant; the remaining units
 * (any layout) run on the general kernel.  Zero for both counts runs
 * everything on the general kernel (same results with SR off).
 * APEXW_MODE_SINGLE runs every unit on the general kernel: both counts must be 0.
 */
int apexw_q8_step(const apexw_tensor* tensors, int32_t n_tensors,
                  const apexw_unit* units, int64_t n_units, int64_t n_fast_units,
                  int64_t n_fast_f32_units, const apexw_hparams* hp, void* stream);

/*
 * Factored second moment (Adafactor-style) for large matrices: the reference's
 * _apply_factored_v_int8_update (apexw/state.py:442-608), used by precision
 * "8bit" (INT8 or packed 6-bit m) and "compact" (16-bit m) with factored_v=True.
 * Per step and tensor, with G = prepared fp32 grad viewed as [rows x cols]:
 *   row  = b2 row + (1-b2) mean_c(G^2)          col = b2 col + (1-b2) mean_r(G^2)
 *          (tensors above 262,144 elements: col = b2 col + ((1-b2)/rows) sum_r(G^2))
 *   nan_to_num(row), nan_to_num(col)
 *   den  = max(sqrt(row / mean(row)) sqrt(col) + eps_scaled, eps)
 *   m    = lerp(m, G, 1-b1)  (dequantized; requantized with the EMA-max scale)
 *   p    = p * wd_factor (where FLAG_WD) - (m / den) * step_size
 * One entry per factored tensor (device array, 32 bytes each).
 */
typedef struct apexw_fv_tensor {
  uint32_t tensor;   /* row of the tensor table */
  int32_t rows;      /* shape[0] */
  int32_t cols;      /* numel / rows */
  uint32_t flags;    /* APEXW_FV_SUM_COLS: the column EMA of a tensor above 262,144 elements */
  int64_t ws;        /* float offset of the tensor's workspace (set by apexw_factored_layout) */
  int32_t band0;     /* first statistics band of the tensor (set by apexw_factored_layout) */
  int32_t cb0;       /* first column block of the tensor (set by apexw_factored_layout) */
} apexw_fv_tensor;

#define APEXW_FV_SUM_COLS 1u
#define APEXW_FV_BAND_ROWS 32   /* rows per statistics band */

/*
 * Host: lay out the workspace of n_fv factored tensors (HOST array, entries in
 * ascending tensor order, rows * cols = the tensor's numel).  Writes ws, band0
 * and cb0 of every entry and the totals; returns the workspace size in floats,
 * or minus a status.
 */
int64_t apexw_factored_layout(apexw_fv_tensor* fv, int32_t n_fv, int64_t* n_bands, int64_t* n_col_blocks);

/*
 * One factored step of every tensor in fv (device array laid out by
 * apexw_factored_layout): statistics, finalisation, then the block update over
 * units (one quantization block each for quantized m, APEXW_COMPACT_UNIT
 * elements for 16-bit m; a unit's `tensor` field is the index of its entry in
 * fv, not a row of the tensor table, so no lookup precedes its loads).  The
 * units are grouped by (parameter dtype, m kind) in the order bf16 / INT8 m,
 * bf16 / 6-bit m, bf16 / bf16 m, fp32 / INT8 m, fp32 / 6-bit m, fp32 / bf16 m,
 * fp16 / INT8 m, fp16 / 6-bit m, fp16 / fp16 m (fp16 parameters: decay and update
 * in fp32, clamped to +-65504, one rounding; 16-bit m in fp16);
 * range_ends (HOST array of APEXW_FV_UNIT_RANGES) holds the end offset of each
 * group (the last is n_units), and each non-empty group runs on its own kernel.
 * workspace: the floats apexw_factored_layout returned.  hp as for the step
 * kernels (mode ignored); APEXW_HP_SR rounds the m codes stochastically.
 */
#define APEXW_FV_UNIT_RANGES 9
int apexw_factored_step(const apexw_tensor* tensors, int32_t n_tensors, const apexw_fv_tensor* fv, int32_t n_fv,
                        int64_t n_bands, int64_t n_col_blocks, const apexw_unit* units, int64_t n_units,
                        const int64_t* range_ends, float* workspace, const apexw_hparams* hp, void* stream);

/*
 * Global-L2 clip coefficient over the grads of the table:
 *   norm_t = dtype_round(||g_t||_2), total = ||(norm_t)||_2,
 *   *coef = min(clip / (total + 1e-6), 1)   (1 when total is not finite).
 * unit_partial: n_units floats of workspace; tensor_norm: n_tensors floats;
 * unit_begin: n_tensors + 1 int64 prefix offsets of each tensor's units.
 * flags: APEXW_HP_SANITIZE to sanitize grads before squaring; APEXW_HP_UNSCALE
 * to take the norm of dtype_round(g * grad_inv_scale) (AMP grads are unscaled
 * before the clip, apexw/optimizer.py:227-237).  amp: when not NULL, the
 * unscale factor is amp->grad_inv_scale, read on the device (apexw_amp_prepare);
 * the same holds for apexw_grad_prepare and apexw_grad_row_means below.
 * APEXW_FLAG_GC descriptors: the norm is that of the centralized grad (its row
 * means from m_scale / block, or from rows[i] when rows is not NULL: 8-bit /
 * ultra tables, one entry per descriptor).
 */
int apexw_grad_clip_coef(const apexw_tensor* tensors, int32_t n_tensors,
                         const apexw_unit* units, int64_t n_units, int64_t unit_size,
                         const int64_t* unit_begin, float* unit_partial, float* tensor_norm,
                         float clip, float grad_inv_scale, uint32_t flags, float* coef,
                         const apexw_amp_dyn* amp, const apexw_row_means* rows, void* stream);

/*
 * apexw_grad_clip_coef without workspace arguments, allocating nothing: the
 * per-unit partial sums and per-tensor norms live in a fixed device array of
 * the library ((APEXW_NOALLOC_CLIP_MAX_UNITS + APEXW_NOALLOC_CLIP_MAX_TENSORS)
 * floats, 32.5 MiB per GPU, held until the process ends: 2^23 units cover an
 * 8B-parameter list in 2048-element units).  The array used is that of the
 * stream's device (hipStreamGetDevice; the current device for the null stream).
 * Same kernels, same result as apexw_grad_clip_coef with rows = NULL.  Returns APEXW_ERR_SIZE,
 * before enqueueing anything, when n_units or n_tensors exceeds its limit.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (two streams, or two host threads) race.
 * Nothing in the array needs to start at zero (every entry is written before
 * it is read within one call).
 */
#define APEXW_NOALLOC_CLIP_MAX_UNITS (1 << 23)
#define APEXW_NOALLOC_CLIP_MAX_TENSORS (1 << 17)
int apexw_grad_clip_coef_noalloc(const apexw_tensor* tensors, int32_t n_tensors,
                                 const apexw_unit* units, int64_t n_units, int64_t unit_size,
                                 const int64_t* unit_begin, float clip, float grad_inv_scale,
                                 uint32_t flags, float* coef, const apexw_amp_dyn* amp, void* stream);

/*
 * Gradient preparation of _prepare_grads (apexw/optimizer.py:204-258) for a
 * group with grad_centralization: writes, per grad, out = g sanitized (NaN -> 0,
 * +-Inf -> +-65504, APEXW_HP_SANITIZE), unscaled (times grad_inv_scale in the
 * grad dtype, APEXW_HP_UNSCALE) and, when row_len > 0, centralized:
 *   out = dtype_round(x - dtype_round(mean over the row of x)),
 * rows being the row_len consecutive elements of each index of dim 0 (the
 * reference's g.sub_(g.mean(dim=(1, ...), keepdim=True)) for dim >= 2).  The
 * step and the clip then read out (the reference also works on a clone).
 */
typedef struct apexw_grad_prep {
  const void* g;        /* source grad, n elements */
  void* out;            /* prepared grad, n elements, same dtype; not aliasing g */
  int64_t n;
  int64_t row_len;      /* centralize rows of this length (n % row_len == 0), or 0 */
  uint32_t dtype;       /* APEXW_F32 / APEXW_BF16 / APEXW_F16 */
  uint32_t reserved;    /* 0 */
} apexw_grad_prep;      /* 40 bytes */

/* Validate one descriptor (host copy) before it is uploaded. */
int apexw_check_grad_prep(const apexw_grad_prep* d);

/* Work units of apexw_grad_prepare for one descriptor: its rows when row_len > 0,
 * else chunks of APEXW_GRAD_PREP_CHUNK elements (unit = index). */
#define APEXW_GRAD_PREP_CHUNK 2048
int64_t apexw_grad_prep_units(const apexw_grad_prep* d);

/* Launch over a device table of descriptors and a unit table ({tensor, unit}
 * entries as for the step), one workgroup per unit. */
int apexw_grad_prepare(const apexw_grad_prep* preps, int32_t n_preps, const apexw_unit* units, int64_t n_units,
                       float grad_inv_scale, uint32_t flags, const apexw_amp_dyn* amp, void* stream);

/*
 * Row means only, for centralization folded into the compact step and the clip
 * (APEXW_FLAG_GC): per descriptor with row_len > 0, out is a float array of
 * n / row_len entries and entry r receives dtype_round(sum of row r of
 * sanitized, unscaled g / row_len) -- the mean apexw_grad_prepare subtracts.
 * Units are the descriptors' rows (unit = row index), one workgroup each.
 * Replaces the same _prepare_grads step as apexw_grad_prepare
 * (apexw/optimizer.py:238-243) without writing a prepared copy of the grads.
 */
int apexw_grad_row_means(const apexw_grad_prep* preps, int32_t n_preps, const apexw_unit* units, int64_t n_units,
                         float grad_inv_scale, uint32_t flags, const apexw_amp_dyn* amp, void* stream);

/* Validate one descriptor (host copy) of apexw_grad_row_means: row_len > 0 divides n, out holds
 * n / row_len floats that do not overlap the grad. */
int apexw_check_row_means(const apexw_grad_prep* d);

/* ------------------------------------------------------------------------- */
/* Muon: Newton-Schulz on the matrix cores                                    */
/* ------------------------------------------------------------------------- */

#define APEXW_GEMM_TILE 256   /* M and N multiple of this */
#define APEXW_GEMM_KTILE 64   /* K multiple of this */
#define APEXW_GEMM_MAX_LD (1 << 22)   /* leading dimensions, elements */

/*
 * Batched bf16 "NT" GEMM on the matrix cores (fp32 accumulation, bf16 output
 * rounded to nearest even):
 *   O[b] = alpha * A[b] . B[b]^T + beta * E[b]
 * A: [m x k] row-major (lda), B: [n x k] row-major (ldb).  E is given
 * transposed: et[j * lde + i] = E[i][j] (needed when beta != 0).  O is written
 * row-major to c ([m x n], ldc) and/or transposed to ct ([n x m], ldct); at
 * least one of them.  m, n multiple of APEXW_GEMM_TILE, k of APEXW_GEMM_KTILE,
 * pointers 16-byte aligned, leading dimensions and batch strides multiples of 8
 * elements and at most APEXW_GEMM_MAX_LD.  Outputs must not alias inputs.
 */
int apexw_gemm_nt_bf16(const void* a, const void* b, const void* et, void* c, void* ct,
                       int32_t m, int32_t n, int32_t k, int32_t lda, int32_t ldb, int32_t lde,
                       int32_t ldc, int32_t ldct, int32_t batch,
                       int64_t stride_a, int64_t stride_b, int64_t stride_e, int64_t stride_c,
                       int64_t stride_ct, float alpha, float beta, void* stream);

/*
 * Grouped launch: the same product for many matrices of different shapes in one
 * persistent launch (one workgroup per CU), replacing the per-shape batched
 * calls of ApexMuon._step_batched / _step_single (apexw/muon.py:593-615,
 * :187-211).  Each problem is one "NT" product with the operand conventions of
 * apexw_gemm_nt_bf16 (a single batch entry).  All problems of a launch write the
 * same outputs (c and/or ct) and either all add beta * E or none does.
 */
typedef struct apexw_gemm_problem {
  const void* a;       /* [m x k] bf16, lda */
  const void* b;       /* [n x k] bf16, ldb ([k x n] with APEXW_GEMM_B_KN) */
  const void* et;      /* E transposed, [n x m], lde; NULL when beta == 0 or APEXW_GEMM_ADD_B */
  void* c;             /* [m x n] output, ldc; NULL = not written */
  void* ct;            /* [n x m] transposed output, ldct; NULL = not written */
  int32_t m, n, k;
  int32_t lda, ldb, lde, ldc, ldct;
  float alpha, beta;
  uint32_t flags;      /* APEXW_GEMM_* bits below */
  uint32_t reserved;   /* 0 */
  /* APEXW_GEMM_APPLY only (else 0): the Muon parameter update fused into the
   * epilogue, p <- p * wd_factor (with APEXW_GEMM_APPLY_WD), then
   * p <- p + neg_lr * O, each rounded to p's dtype, for every element of
   * p [p_rows x p_cols] (row-major); O covers p (APEXW_GEMM_APPLY_T: O = p^T). */
  void* p;
  int32_t p_dtype;     /* APEXW_F32 / APEXW_BF16 / APEXW_F16 */
  int32_t p_rows, p_cols;
  float wd_factor, neg_lr;
  uint32_t reserved2;  /* 0 */
} apexw_gemm_problem;  /* 120 bytes */

/* The product is symmetric (A A^T, or c A A + b A with A symmetric): m == n,
 * a == b, and ct == c with ldct == ldc.  Only tiles on and above the diagonal
 * are computed; each off-diagonal tile is also stored mirrored, so c receives
 * the whole matrix.  E, when added, must be symmetric. */
#define APEXW_GEMM_SYM 1u
/* B is given as [k x n] row-major (ldb >= n): O = alpha A B + beta E.  Not with
 * APEXW_GEMM_SYM; only row-major output (ct NULL). */
#define APEXW_GEMM_B_KN 2u
/* The addend is the B operand read at K = row: E[i][j] = B[j][i] ([n x k] B) or
 * B[i][j] (APEXW_GEMM_B_KN), as in X' = B X + a X.  Requires alpha == 1,
 * m <= k, beta != 0 and et NULL; it is accumulated on the matrix cores (beta
 * as two bf16 parts, within 2^-18 of beta) instead of read in the epilogue. */
#define APEXW_GEMM_ADD_B 4u
/* The epilogue applies the Muon update to p (fields above) instead of, or,
 * when c is not NULL, besides writing O: ApexMuon's decoupled decay and
 * scaled orthogonalised update (apexw/muon.py:852-858) on the last
 * Newton-Schulz product, with no separate pass over O.  Only with
 * APEXW_GEMM_ADD_B (the X' = B X + a X product): with APEXW_GEMM_B_KN ct is NULL;
 * with X^T as the [n x k] operand ct may receive O^T as well. */
#define APEXW_GEMM_APPLY 8u
#define APEXW_GEMM_APPLY_T 16u   /* O is p transposed (a tall parameter's wide work matrix) */
#define APEXW_GEMM_APPLY_WD 32u  /* multiply p by wd_factor first */
/* Every matrix of the problem (a, b, et, c, ct) is stored in 32 x 32 panels:
 * element (r, c) of a matrix whose leading dimension is ld sits at
 * (r / 32) * 32 * ld + (c / 32) * 1024 + (r % 32) * 32 + c % 32 (panels of 1024
 * contiguous elements, row-major inside and in row-major order).  Every K stage
 * of an operand is then a run of whole 128-byte lines.  Leading dimensions must
 * be multiples of 32.  p (APEXW_GEMM_APPLY) stays row-major. */
#define APEXW_GEMM_PANEL 64u

/* epilogue kinds of a grouped launch (bit mask) */
#define APEXW_GEMM_OUT_C 1   /* row-major output */
#define APEXW_GEMM_OUT_CT 2  /* transposed output */
#define APEXW_GEMM_ADD 4     /* beta * E added */
#define APEXW_GEMM_KIND_NN 8 /* B given as [k x n] (APEXW_GEMM_B_KN) */
#define APEXW_GEMM_KIND_PANEL 16 /* matrices in 32 x 32 panels (APEXW_GEMM_PANEL) */

/* Tile queues of a grouped launch: one per XCD of MI355X. */
#define APEXW_GEMM_QUEUES 8

/* Output tiles (work items) of a grouped launch, or minus an apexw_status when
 * a problem is invalid. */
int64_t apexw_gemm_grouped_items(const apexw_gemm_problem* problems, int32_t n_problems);

/*
 * Host-side: validate the problems (a host copy of the table that will be
 * uploaded) and build the tile queues: items[*n_items_out] (capacity n_items,
 * at least twice apexw_gemm_grouped_items) and
 * queue_offsets[APEXW_GEMM_QUEUES + 1]; queue q is
 * items[queue_offsets[q] .. queue_offsets[q + 1]).  Each problem's tiles, in
 * locality order (bands of 4 tile rows), are cut into one contiguous band per
 * queue (so every XCD works on the same matrix at once), the remainders rotated
 * across queues to balance them; longest tiles first within a queue.  With
 * cus_per_queue > 0 (the CUs of one XCD: the device's CU count / 8), the last
 * tiles of a queue may be split into two 128-row halves, as many as minimise
 * the queue's simulated makespan, so that the last round fills the XCD; 0
 * keeps whole tiles.  *n_workgroups receives the grid size of the launch
 * (APEXW_GEMM_QUEUES x the longest queue) and *kind the epilogue kind.  At most
 * 256 problems, 2048 tiles per side.
 */
int apexw_gemm_grouped_schedule(const apexw_gemm_problem* problems, int32_t n_problems, uint32_t* items,
                                int64_t n_items, int32_t cus_per_queue, int64_t* n_items_out,
                                int32_t* queue_offsets, int32_t* n_workgroups, int32_t* kind);

/*
 * Run a grouped launch: one workgroup per tile; workgroup b computes tile
 * b / APEXW_GEMM_QUEUES of queue b % APEXW_GEMM_QUEUES (workgroups are
 * dispatched round-robin over the XCDs, so each XCD works through one queue).
 * problems, items and queue_offsets are device copies of the arrays validated
 * and built by apexw_gemm_grouped_schedule, n_workgroups and kind its outputs;
 * like the tensor tables of the step, they are trusted as built.  amp: NULL,
 * or GradScaler's step read on the device (apexw_amp_prepare): every
 * workgroup returns before any write when amp->skip.
 */
int apexw_gemm_nt_grouped(const apexw_gemm_problem* problems, const uint32_t* items, const int32_t* queue_offsets,
                          int32_t n_workgroups, int32_t kind, const apexw_amp_dyn* amp, void* stream);

/* fp32 workspace (floats) apexw_muon_prepare needs for a [rows x cols] matrix. */
/* Layout of a Newton-Schulz work matrix in apexw_muon_prepare / apexw_muon_apply:
 * row-major with leading dimension ld, or 32 x 32 panels as APEXW_GEMM_PANEL
 * describes (ld a multiple of 32; the rows the panels cover rounded up to 32). */
#define APEXW_LAYOUT_ROWS 0
#define APEXW_LAYOUT_PANEL 1
int64_t apexw_muon_workspace_floats(int64_t rows, int64_t cols);

/*
 * Muon momentum and Newton-Schulz input for one [rows x cols] parameter:
 *   buf = buf * mu + (1 - mu) * g        (fp32 buffer; g = dtype_round(g * grad_inv_scale)
 *                                         when grad_inv_scale != 1 (AMP), then sanitized
 *                                         NaN -> 0, +-Inf -> +-65504; g dtype F32/BF16/F16)
 *   s   = buf, or lerp(g, buf, mu) when nesterov
 *   X   = bf16(bf16(s) / bf16(bf16(||bf16(s)||_F) + eps))
 * X is written as the wide work matrix [min x max] to x (ldx) and, when xt is
 * not NULL, as its transpose [max x min] to xt (ldxt): when rows > cols the
 * work matrix is s^T.  Both in `layout` (APEXW_LAYOUT_ROWS or _PANEL, the latter
 * for grouped products with APEXW_GEMM_PANEL).  Elements of x / xt outside the
 * matrix are not written (keep them zero).  amp (NULL or 16-byte aligned): GradScaler's step read on
 * the device (apexw_amp_prepare), in place of the host's found_inf.item() /
 * grad_scale.reciprocal().item() (apexw/muon.py:557-577): nothing is written
 * when amp->skip, and amp->grad_inv_scale replaces grad_inv_scale.  The same
 * argument of apexw_muon_apply, apexw_muon_coordwise and apexw_gemm_nt_grouped
 * skips the rest of the step.
 */
int apexw_muon_prepare(float* buf, const void* g, int32_t g_dtype, int64_t rows, int64_t cols,
                       float mu, float one_minus_mu, int32_t nesterov, float eps, float grad_inv_scale,
                       void* x, void* xt, int64_t ldx, int64_t ldxt, int32_t layout, float* workspace,
                       const apexw_amp_dyn* amp, void* stream);

/*
 * p = round(round(p * wd_factor) + neg_lr_eff * U)   (the decay only if apply_wd)
 * with U the bf16 Newton-Schulz result in p's [rows x cols] shape (leading
 * dimension ldu, stored in `layout`: APEXW_LAYOUT_ROWS or _PANEL), or, when
 * u_transposed, given as U^T [cols x rows] (the wide work matrix of a tall
 * parameter); p dtype F32/BF16/F16, rounded to nearest even.
 */
int apexw_muon_apply(void* p, int32_t p_dtype, const void* u, int64_t rows, int64_t cols, int64_t ldu,
                     int32_t layout, int32_t u_transposed, float wd_factor, int32_t apply_wd, float neg_lr_eff,
                     const apexw_amp_dyn* amp, void* stream);

/*
 * Coordinate-wise Muon update of one parameter that Newton-Schulz does not take
 * (a vector, or a matrix with a dimension under 16): ApexMuon._step_single's
 * fallback (apexw/muon.py:775-799, :841-858).  n elements, contiguous:
 *   g   = nan_to_num(dtype_round(g * grad_inv_scale), 0, +-65504)
 *   buf = buf * mu + (1 - mu) * g                  (fp32)
 *   s   = buf, or lerp(g, buf, mu) when nesterov
 *   U   = s / (std(s, unbiased=False) + 1e-7)     (n == 1: s / (|s| + 1e-7))
 *   p   = round(round(p * wd_factor) + neg_lr * round(U))   (the decay only if apply_wd)
 * neg_lr = -lr * 0.05 for the reference's fallback scale.  One workgroup.
 */
int apexw_muon_coordwise(float* buf, const void* g, int32_t g_dtype, void* p, int32_t p_dtype, int64_t n, float mu,
                         float one_minus_mu, int32_t nesterov, float grad_inv_scale, float wd_factor,
                         int32_t apply_wd, float neg_lr, const apexw_amp_dyn* amp, void* stream);

/* ------------------------------------------------------------------------- */
/* Optimizer state across precision modes                                     */
/* ------------------------------------------------------------------------- */

/*
 * One parameter's moment buffers (device pointers), for resuming a checkpoint
 * in another precision mode.  Replaces nothing in the reference: its
 * load_state_dict keeps the saved layout (apexw/optimizer.py:2487-2572), so a
 * state saved by one mode cannot be stepped by another; ApexW.load_state_dict
 * here converts it with these two calls.
 *   APEXW_STATE_DENSE: m and v in the MDT / VDT dtypes of flags (F32 / BF16 /
 *     F16), v with n/4 entries when APEXW_FLAG_QUAD; block = 0.
 *   APEXW_STATE_Q8: m = NF4 codes (APEXW_FLAG_NF4: uint8, two per byte, even
 *     element in the high nibble, (n+1)/2 bytes) or INT8 codes (n bytes), v =
 *     log-uint8 codes (n/4 with APEXW_FLAG_QUAD, else n), m_scale / v_scale one
 *     fp32 per block of `block` elements (<= 2048; a multiple of 8 with NF4 or
 *     QUAD; the quad v block is block/4 codes under the same scale index).
 */
#define APEXW_STATE_DENSE 0u
#define APEXW_STATE_Q8 1u
typedef struct apexw_state_layout {
  void* m;
  void* v;
  float* m_scale;
  float* v_scale;
  int64_t n;
  uint32_t kind;
  uint32_t flags;     /* APEXW_FLAG_MDT/VDT fields (dense), APEXW_FLAG_QUAD, APEXW_FLAG_NF4 (q8) */
  uint32_t block;
  uint32_t reserved;  /* 0 */
} apexw_state_layout;   /* 56 bytes */

/*
 * Expand the state s (HOST descriptor of device buffers) to fp32 moments:
 * m_out and v_out receive n floats each (a quad v value on each of its 4
 * elements); 8-bit codes decode as codebook value (NF4), code (INT8) or
 * 2^((q-1) 24/254 - 24) (log-uint8, 0 for q = 0) times the block scale.
 */
int apexw_state_decode(const apexw_state_layout* s, float* m_out, float* v_out, void* stream);

/*
 * Build the state s from fp32 moments m_in, v_in (n floats each): dense
 * buffers rounded to nearest even (quad v: the mean of each 4, summed
 * pairwise); 8-bit codes and block scales from the values alone, as the
 * reference's quantizers with no previous scale (apexw/quantization.py:66-126,
 * :277-357, :381-448), round to nearest.
 */
int apexw_state_encode(const apexw_state_layout* s, const float* m_in, const float* v_in, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* APEXW_HIP_H */
