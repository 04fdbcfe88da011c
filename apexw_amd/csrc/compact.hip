// Compact-precision fused multi-tensor AdamW step (gfx950).
//
// One launch covers every tensor of a parameter group.  The chunk table splits
// tensors into units of APEXW_COMPACT_UNIT (2048) elements; each wavefront takes
// units in a grid-stride loop, so a launch of a few thousand workgroups keeps
// all 256 CUs busy whatever the tensor sizes.  A lane owns 4 groups of 8
// consecutive elements (16-byte loads for bf16, 2x16-byte for fp32) spaced one
// wave-width apart, so every load/store instruction of a wave touches one
// contiguous 1-2 KiB span.
//
// The arithmetic restates the reference's CPU op sequence (rounding to the
// storage dtype after each torch op):
//   cold   = ApexW._multi_tensor_step   (apexw/optimizer.py:5297-5887)
//   replay = FastExecutionPlan.execute_foreach (apexw/optimizer.py:1069-1341)
//   native = torch._fused_adamw_ as called by _fused_step (apexw/optimizer.py:4737-4835)
//   single = ApexW._step_single_param_fused, compact branch (apexw/optimizer.py:2458-2471)
#include "common.h"

namespace {

constexpr int kWaves = 4;        // wavefronts per workgroup
constexpr int kGroups = 4;       // 8-element groups per lane per unit

struct Ctx {
  const apexw_hparams* hp;
  float coef;
  uint32_t key;
  uint32_t tflags;
  float vscale, vscale_sqrt;   // the tensor's dynamic fp16-v scale (APEXW_FLAG_VSCALE), else 1
  float cq;                    // cautious: the tensor's 1 / mean(mask) (caut_q), else unused
};

// torch.maximum of two second moments: NaN when either is NaN
APEXW_DEV float max_nan(float a, float b) { return (b > a || b != b) ? b : a; }

// A 16-bit parameter stored through the reference's fp32 -> 16-bit copy
// (_copy_fp32_to_16bit_sr_ without SR): fp16 is clamped to its range first.
template <int PD> APEXW_DEV float store_p(float x) {
  if constexpr (PD == APEXW_F16) return rnd<PD>(clamp_f16_range(x));
  else return rnd<PD>(x);
}

// sanitize (san), AMP unscale (in place on the grads: _multi_tensor_step,
// apexw/optimizer.py:5530-5537, or _prepare_grads before a clip), grad
// centralization (g - its row's mean, in the grad dtype, when gc), clip: the
// order of _prepare_grads (apexw/optimizer.py:204-258)
template <int GD> APEXW_DEV float prep_grad(float g, const Ctx& c, bool san, bool gc, float mean) {
  if (san) g = sanitize<GD>(g);
  if (c.hp->flags & APEXW_HP_UNSCALE) g = rnd<GD>(g * c.hp->grad_inv_scale);
  if (gc) g = rnd<GD>(g - mean);
  if (c.hp->flags & APEXW_HP_CLIP) g = rnd<GD>(g * c.coef);
  return g;
}

// Row means of a centralized grad for the 8 elements from e0: the tensor's
// row_len (t.block) elements form a row; t.m_scale holds each row's mean.
APEXW_DEV void row_means8(const apexw_tensor& t, int64_t e0, float (&mean)[8]) {
  const int64_t rl = (int64_t)t.block;
  const float* means = t.m_scale;
  const int64_t rows = t.n / rl;
  if (rl >= 8) {
    // at most one row boundary inside the 8 elements
    const int64_t row = e0 / rl, col = e0 - row * rl;
    const float m0 = means[row];
    const float m1 = (col + 8 > rl && row + 1 < rows) ? means[row + 1] : m0;
#pragma unroll
    for (int j = 0; j < 8; ++j) mean[j] = col + j < rl ? m0 : m1;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t r = (e0 + j) / rl;
      mean[j] = means[r < rows ? r : rows - 1];
    }
  }
}

// True when any of the 8 grads is NaN or +-Inf (g * 0 is NaN exactly then): the
// per-element sanitize runs only for such a lane (rare), one fma per element otherwise.
APEXW_DEV bool any_nonfinite8(const float (&g)[8]) {
  float t = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) t = fmaf(g[j], 0.0f, t);
  return !(t == t);
}

// Quotient and square root: round to nearest (IEEE) without SR; with SR the
// hardware reciprocal and square root (within 1 ulp), whose last-bit error is far
// below the 2^-16-relative noise the stochastic rounding adds.
template <bool SR> APEXW_DEV float q_div(float x, float y) {
  if constexpr (SR) return x * __builtin_amdgcn_rcpf(y);
  else return x / y;
}
template <bool SR> APEXW_DEV float q_sqrt(float x) {
  if constexpr (SR) return __builtin_amdgcn_sqrtf(x);
  else return sqrtf(x);
}

// First moment of the cold and replayed orders: the cold step's 16-bit-moment
// branch = mul then add-with-alpha (two roundings), its fp32-moment branch = one
// lerp on the grads cast to fp32 (apexw/optimizer.py:5778-5781); the replay = one
// lerp when grad and moment dtypes match, else mul then add (:1228-1238).
template <int GD, int MD> APEXW_DEV void m_update8(float (&m)[8], const float (&g)[8], const apexw_hparams& hp) {
  constexpr bool kLerpCold = MD == APEXW_F32, kLerpReplay = GD == MD;
  if (hp.mode == APEXW_MODE_REPLAY ? kLerpReplay : kLerpCold) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float d = g[j] - m[j];
      m[j] = rnd<MD>((hp.flags & APEXW_HP_LERP_HI) ? fmaf(hp.lerp_coef, d, g[j]) : fmaf(hp.lerp_coef, d, m[j]));
    }
  } else {
    const float b1_m = rnd<MD>(hp.beta1);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float m1 = rnd<MD>(m[j] * b1_m);
      m[j] = rnd<MD>(fmaf(hp.one_minus_beta1, g[j], m1));
    }
  }
}

// The slow first moment of beta3 (APEXW_HP_SLOW), beside m and in its dtype, in the same
// order as m: lerp with weight 1 - beta3 where m_update8 lerps, else mul by beta3 rounded to
// m's dtype then add (1 - beta3) g (apexw/optimizer.py:5763-5765, :5781, :1232-1238)
template <int GD, int MD> APEXW_DEV void slow_update8(float (&s)[8], const float (&g)[8], const apexw_hparams& hp) {
  constexpr bool kLerpCold = MD == APEXW_F32, kLerpReplay = GD == MD;
  if (hp.mode == APEXW_MODE_REPLAY ? kLerpReplay : kLerpCold) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float d = g[j] - s[j];
      s[j] = rnd<MD>((hp.flags & APEXW_HP_LERP3_HI) ? fmaf(hp.lerp3_coef, d, g[j]) : fmaf(hp.lerp3_coef, d, s[j]));
    }
  } else {
    const float b3_m = rnd<MD>(hp.beta3);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float s1 = rnd<MD>(s[j] * b3_m);
      s[j] = rnd<MD>(fmaf(hp.one_minus_beta3, g[j], s1));
    }
  }
}

// cautious (APEXW_HP_CAUTIOUS): the mask g m >= 0 of one element (g prepared, m
// updated), its product formed where the reference forms it: in fp32 for quad v
// (apexw/optimizer.py:5728, :1272) and the cold order (:5851-5853), in the grads'
// dtype after m is cast to it for the replayed order (:1322-1325)
template <int GD, bool QUAD> APEXW_DEV bool caut_mask(float g, float m, int mode) {
  if (!QUAD && mode == APEXW_MODE_REPLAY) return rnd<GD>(g * rnd<GD>(m)) >= 0.0f;
  return g * m >= 0.0f;
}

// 1 / mean(mask) of a tensor with cnt of its n mask bits set, as the reference forms
// it: the mean clamped below by 1e-3, then the quotient, in fp32 for quad v and in
// the parameter's dtype otherwise (the mask is cast to it), each rounded to it
// (torch's CPU mean of a 0/1 mask is fl32(cnt) / fl32(n) rounded to the mask dtype)
APEXW_DEV float caut_q(unsigned long long cnt, int64_t n, bool quad, uint32_t pd) {
  const float mean = (float)cnt / (float)n;
  if (quad || pd == APEXW_F32) return 1.0f / fmaxf(mean, 1e-3f);
  if (pd == APEXW_BF16) return rnd<APEXW_BF16>(1.0f / fmaxf(rnd<APEXW_BF16>(mean), rnd<APEXW_BF16>(1e-3f)));
  return rnd<APEXW_F16>(1.0f / fmaxf(rnd<APEXW_F16>(mean), rnd<APEXW_F16>(1e-3f)));
}

// The dtype torch gives the cold order's cautious numerator m * mask: m (upcast to
// fp32 for an fp32 parameter, optimizer.py:5834-5838) times the mask in the
// parameter's dtype, by type promotion
template <int PD, int MD> constexpr int caut_cold_dtype() {
  constexpr int nd = (PD == APEXW_F32 && MD != APEXW_F32) ? APEXW_F32 : MD;
  return nd == PD ? PD : APEXW_F32;
}

// p, g, m: 8 elements; v: 8 entries (non-quad) or 2 (quad).  cnt <= 8 valid.
// e0 is the element index of slot 0 within the tensor (RNG counter).
// SR: the launch's APEXW_HP_SR flag (a template parameter so that each path
// compiles to its own code); APEXW_HP_SR_V implies it.
// VAR: the launch may carry nesterov, cautious, amsgrad, lion or beta3 (APEXW_HP_NESTEROV /
// _CAUTIOUS / _AMSGRAD / _LION / _SLOW); the plain instantiation compiles without them and
// keeps its registers for the rest.  x: amsgrad's running max of v; ms: beta3's slow moment
// (8 entries each, non-quad only).
template <int PD, int GD, int MD, int VD, bool QUAD, bool SR, bool VAR>
APEXW_DEV void update8(float (&p)[8], float (&g)[8], float (&m)[8], float (&v)[8], float (&x)[8], float (&ms)[8],
                       int cnt, uint32_t e0, const Ctx& c, bool gc, const float (&mean)[8], bool ams, bool slow,
                       int tj) {
  const apexw_hparams& hp = *c.hp;
  constexpr bool sr = SR;
  const bool srv = SR && (hp.flags & APEXW_HP_SR_V);
  const bool wd = c.tflags & APEXW_FLAG_WD;
  // 32 random bits per element (bits 0-15 round p, bits 16-31 round v): a xorshift32
  // stream per lane and 8-element group, seeded by a keyed hash of the group's first
  // element index
  uint32_t rnd_bits[8];
  if constexpr (SR) {
    uint32_t rs = mix32(c.key + e0) | 1u;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      rs ^= rs << 13;
      rs ^= rs >> 17;
      rs ^= rs << 5;
      rnd_bits[j] = rs;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) rnd_bits[j] = 0u;
  }
  const bool san = (hp.flags & APEXW_HP_SANITIZE) && any_nonfinite8(g);
#pragma unroll
  for (int j = 0; j < 8; ++j) g[j] = prep_grad<GD>(g[j], c, san, gc, mean[j]);
  // ams (amsgrad): the denominator's v is max(max_v, v') (torch._foreach_maximum_ after
  // the v update, apexw/optimizer.py:5788-5790, :1253-1255; inside torch._fused_adamw_ for
  // the native mode)

  if constexpr (VAR && !QUAD) {
    if (hp.flags & APEXW_HP_LION) {
      // lion (the cold and the replayed order alike, apexw/optimizer.py:5677-5683,
      // :1214-1225): the grads cast to m's dtype; u = lerp(g', m, beta1) rounded to it;
      // p += -lr * sign(u), the scalar rounded to p's dtype when p and u share a 16-bit
      // dtype (torch's same-dtype add with alpha, see tj below: the product with a sign is
      // exact either way); m = lerp(m, g', 1 - beta2)
      constexpr bool kAlpha16 = PD == MD && PD != APEXW_F32;
      const float alpha = kAlpha16 ? rnd<PD>(-hp.gain_hi) : -hp.gain_hi;
      const float wd_l = rnd<PD>(hp.wd_factor);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float pw = wd ? rnd<PD>(p[j] * wd_l) : p[j];
        const float gm = rnd<MD>(g[j]);
        const float d = m[j] - gm;
        const float u = rnd<MD>((hp.flags & APEXW_HP_LOOK_HI) ? fmaf(hp.look_coef, d, m[j])
                                                               : fmaf(hp.look_coef, d, gm));
        const float sg = u > 0.0f ? 1.0f : (u < 0.0f ? -1.0f : 0.0f);
        p[j] = rnd<PD>(pw + alpha * sg);
        m[j] = rnd<MD>((hp.flags & APEXW_HP_LERP_HI) ? fmaf(hp.lerp_coef, -d, gm) : fmaf(hp.lerp_coef, -d, m[j]));
      }
      return;
    }
  }

  if constexpr (!QUAD) {
    if (hp.mode == APEXW_MODE_SINGLE) {
      // p.mul_(wd) in the parameter dtype (fp32 scalar), fp32 moments
      // (mul_ then add_ with alpha: one FMA; addcmul_: one FMA), p.addcdiv_ in
      // fp32 rounded once, m and v rounded once on store
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float pf = wd ? rnd<PD>(p[j] * hp.wd_factor) : p[j];
        const float mf = fmaf(hp.one_minus_beta1, g[j], m[j] * hp.beta1);
        const float vf = fmaf(hp.one_minus_beta2 * g[j], g[j], v[j] * hp.beta2);
        const float den = sqrtf(vf) + hp.eps_scaled;
        p[j] = rnd<PD>(pf + (-hp.step_size * mf) / den);
        m[j] = rnd<MD>(mf);
        v[j] = rnd<VD>(vf);
      }
      return;
    }
  }

  if (hp.mode == APEXW_MODE_NATIVE) {
    // torch._fused_adamw_: fp32 math on loaded values, one rounding per stored tensor.
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float pf = wd ? p[j] * hp.wd_factor : p[j];
      float mf = (hp.flags & APEXW_HP_LERP_HI) ? fmaf(hp.lerp_coef, g[j] - m[j], g[j])
                                                : fmaf(hp.lerp_coef, g[j] - m[j], m[j]);
      float vf = v[j] * hp.beta2 + (hp.one_minus_beta2 * g[j]) * g[j];
      float vs = vf;
      if (ams) {
        // the fp32 max feeds the denominator; the stored max is rounded
        vs = max_nan(x[j], vf);
        x[j] = rnd<VD>(vs);
      }
      float den = sqrtf(vs) / hp.bc2_sqrt + hp.eps;
      pf = pf - (hp.step_size * mf) / den;
      p[j] = rnd<PD>(pf);
      m[j] = rnd<MD>(mf);
      v[j] = rnd<VD>(vf);
    }
    return;
  }

  // Same-dtype foreach ops with a Python scalar (_foreach_mul_, _foreach_add_)
  // round the scalar to the tensor dtype first on torch's CPU path, so the
  // 16-bit tensors see bf16(beta1), bf16(beta2), bf16(1 - lr*wd), bf16(eps).
  const float wd_p = rnd<PD>(hp.wd_factor), b2_v = rnd<VD>(hp.beta2);
  // a dynamically scaled v (fp16): the EMA adds (1 - beta2) * scale * g^2 (the scale is
  // a power of two, so the product is exact) and the denominator is
  // (sqrt(v) + eps_scaled * sqrt(scale)) / sqrt(scale) (apexw/optimizer.py:5691-5721,
  // :5799-5816); the replay with fp16 in the subgroup clamps it below by eps (:1264-1265,
  // :1310-1311)
  const bool scaled = c.vscale != 1.0f;
  const float omb2 = hp.one_minus_beta2 * c.vscale;
  const float eps_v = rnd<VD>(scaled ? hp.eps_scaled * c.vscale_sqrt : hp.eps_scaled);
  const float sqrt_scale_v = rnd<VD>(c.vscale_sqrt);
  constexpr bool kFp16 = PD == APEXW_F16 || MD == APEXW_F16 || VD == APEXW_F16;
  const bool clamp_den = kFp16 && hp.mode == APEXW_MODE_REPLAY;
  const float eps_floor = rnd<VD>(hp.eps);
  if (wd) {
#pragma unroll
    for (int j = 0; j < 8; ++j) p[j] = rnd<PD>(p[j] * wd_p);
  }
  m_update8<GD, MD>(m, g, hp);
  if (slow) slow_update8<GD, MD>(ms, g, hp);
  const bool p16 = PD != APEXW_F32;
  // nesterov (the cold and the replayed foreach orders): quad tensors take
  // lerp(g, m, beta1) as the numerator (apexw/optimizer.py:5732-5733, :1276-1277,
  // look_coef / APEXW_HP_LOOK_HI as the 8-bit lookahead); the others two addcdiv
  // passes, p += (gain_hi * m) / d then p += (gain_lo * g) / d with gain_hi =
  // -step_size * beta1 and gain_lo = -step_size * (1 - beta1), each rounded to p's
  // dtype and never stochastic (:5865-5877, :1329-1331)
  const bool nest = VAR && (hp.flags & APEXW_HP_NESTEROV);
  // cautious: m times the mask over its mean (c.cq), in fp32 for quad v (then the usual
  // quad update); otherwise in the dtypes caut_mask / caut_cold_dtype give, then one
  // addcdiv rounded to p's dtype, never stochastic (apexw/optimizer.py:5847-5864,
  // :1321-1328)
  const bool caut = VAR && (hp.flags & APEXW_HP_CAUTIOUS);
  if constexpr (QUAD) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      if (4 * q >= cnt) break;
      const int b = 4 * q;
      float s = g[b] * g[b];
      s = s + g[b + 1] * g[b + 1];
      s = s + g[b + 2] * g[b + 2];
      s = s + g[b + 3] * g[b + 3];
      const float gq = s * 0.25f;
      float vq;
      if (srv) {
        vq = sr_round<VD>(fmaf(omb2, gq, v[q] * hp.beta2), rnd_bits[b] >> 16);
      } else {
        float v1 = rnd<VD>(v[q] * b2_v);
        vq = rnd<VD>(fmaf(omb2, gq, v1));
      }
      v[q] = vq;
      float den = rnd<VD>(q_sqrt<SR>(vq));
      den = rnd<VD>(den + eps_v);
      if (scaled) den = rnd<VD>(den / sqrt_scale_v);
      if (clamp_den) den = fmaxf(den, eps_floor);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = b + i;
        float num = m[j];
        if (caut) {
          num = m[j] * (caut_mask<GD, true>(g[j], m[j], hp.mode) ? c.cq : 0.0f);
        } else if (nest) {
          const float d = m[j] - g[j];
          num = (hp.flags & APEXW_HP_LOOK_HI) ? fmaf(hp.look_coef, d, m[j]) : fmaf(hp.look_coef, d, g[j]);
        }
        const float delta = q_div<SR>(num, den) * hp.step_size;
        const float x = p[j] - delta;
        p[j] = !p16 ? x : (sr ? sr_round<PD>(x, rnd_bits[j]) : store_p<PD>(x));
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float vf;
      if (srv) {
        vf = sr_round<VD>(fmaf(omb2 * g[j], g[j], v[j] * hp.beta2), rnd_bits[j] >> 16);
      } else {
        float v1 = rnd<VD>(v[j] * b2_v);
        vf = rnd<VD>(fmaf(omb2 * g[j], g[j], v1));
      }
      v[j] = vf;
      if (ams) {
        // both sides hold VD values: the max is exact
        vf = max_nan(x[j], vf);
        x[j] = vf;
      }
      float den = rnd<VD>(q_sqrt<SR>(vf));
      den = rnd<VD>(den + eps_v);
      if (scaled) den = rnd<VD>(den / sqrt_scale_v);
      if (clamp_den) den = fmaxf(den, eps_floor);
      if (slow) {
        // AdEMAMix: m + slow_ratio s, upcast to fp32 in the cold order for an fp32 p over
        // 16-bit m (apexw/optimizer.py:5834-5845), else in m's dtype with the ratio rounded
        // to a 16-bit m dtype (torch's same-dtype add with alpha; replay :1332-1334); then one
        // round-to-nearest addcdiv, nesterov ignored
        constexpr bool kUp = PD == APEXW_F32 && MD != APEXW_F32;
        float num;
        if ((kUp && hp.mode != APEXW_MODE_REPLAY) || MD == APEXW_F32) {
          num = fmaf(hp.slow_ratio, ms[j], m[j]);
        } else {
          const float r16 = rnd<MD>(hp.slow_ratio);
          num = rnd<MD>(j < tj ? fmaf(r16, ms[j], m[j]) : m[j] + rnd<MD>(r16 * ms[j]));
        }
        p[j] = rnd<PD>(p[j] + (-hp.step_size * num) / den);
      } else if (caut) {
        const bool replay = hp.mode == APEXW_MODE_REPLAY;
        const float num = replay ? rnd<GD>(m[j]) : m[j];
        float nf = num * (caut_mask<GD, false>(g[j], m[j], hp.mode) ? c.cq : 0.0f);
        // the replay's m (cast to the grad dtype) times the mask (parameter dtype): their promotion
        nf = replay ? rnd<(GD == PD ? PD : APEXW_F32)>(nf) : rnd<caut_cold_dtype<PD, MD>()>(nf);
        p[j] = rnd<PD>(p[j] + (-hp.step_size * nf) / den);
      } else if (nest) {
        const float p1 = rnd<PD>(p[j] + (hp.gain_hi * m[j]) / den);
        p[j] = rnd<PD>(p1 + (hp.gain_lo * g[j]) / den);
      } else if (!p16) {
        p[j] = p[j] + q_div<SR>(-hp.step_size * m[j], den);
      } else if (sr) {
        p[j] = sr_round<PD>(p[j] - q_div<SR>(m[j], den) * hp.step_size, rnd_bits[j]);
      } else if (hp.mode == APEXW_MODE_REPLAY) {
        p[j] = store_p<PD>(p[j] - (m[j] / den) * hp.step_size);
      } else {
        p[j] = rnd<PD>(p[j] + (-hp.step_size * m[j]) / den);
      }
    }
  }
}

// Group k (512 elements, 8 per lane) of the unit starting at element `start`.
// vmax: amsgrad's running max of v for this tensor (hparams.max_v), else NULL.
template <int PD, int GD, int MD, int VD, bool QUAD, bool SR, bool VAR>
APEXW_DEV void compact_group(const apexw_tensor& t, int64_t start, int k, const Ctx& c, void* vmax, void* mslow) {
  const int64_t n = t.n;
  const int lane = lane_id();
  const bool vec = !(c.tflags & APEXW_FLAG_SCALAR);
  {
    const int64_t e0 = start + (int64_t)(k * 64 + lane) * 8;
    if (e0 >= n) return;
    const int cnt = (int)((n - e0) < 8 ? (n - e0) : 8);
    float p[8], g[8], m[8], v[8], x[8], ms[8];
    const bool full = vec && cnt == 8;
    const bool ams = VAR && !QUAD && vmax != nullptr;
    const bool slow = VAR && !QUAD && mslow != nullptr;
    // lion keeps no second moment: v is neither read nor written
    const bool lion = VAR && !QUAD && (c.hp->flags & APEXW_HP_LION);
    if (full) {
      load8<PD>(t.p, e0, p);
      load8<GD>(t.g, e0, g);
      load8<MD>(t.m, e0, m);
      if (slow) load8<MD>(mslow, e0, ms);
      if constexpr (QUAD) {
        if constexpr (VD == APEXW_F32) {
          const u32x2 w = __builtin_nontemporal_load((const u32x2*)((const float*)t.v + (e0 >> 2)));
          v[0] = __uint_as_float(w.x);
          v[1] = __uint_as_float(w.y);
        } else {
          const uint32_t w = __builtin_nontemporal_load((const uint32_t*)((const uint16_t*)t.v + (e0 >> 2)));
          v[0] = VD == APEXW_BF16 ? bf16_bits_to_f32(w & 0xFFFFu) : f16_bits_to_f32(w & 0xFFFFu);
          v[1] = VD == APEXW_BF16 ? __uint_as_float(w & 0xFFFF0000u) : f16_bits_to_f32(w >> 16);
        }
      } else if (!lion) {
        load8<VD>(t.v, e0, v);
        if (ams) load8<VD>(vmax, e0, x);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool ok = j < cnt;
        p[j] = ok ? load1<PD>(t.p, e0 + j) : 0.0f;
        g[j] = ok ? load1<GD>(t.g, e0 + j) : 0.0f;
        m[j] = ok ? load1<MD>(t.m, e0 + j) : 0.0f;
        if constexpr (!QUAD) v[j] = (ok && !lion) ? load1<VD>(t.v, e0 + j) : 0.0f;
        x[j] = (ams && ok) ? load1<VD>(vmax, e0 + j) : 0.0f;
        ms[j] = (slow && ok) ? load1<MD>(mslow, e0 + j) : 0.0f;
      }
      if constexpr (QUAD) {
        v[0] = cnt >= 4 ? load1<VD>(t.v, e0 >> 2) : 0.0f;
        v[1] = cnt >= 8 ? load1<VD>(t.v, (e0 >> 2) + 1) : 0.0f;
      }
    }
    const bool gc = c.tflags & APEXW_FLAG_GC;
    float mean[8];
    if (gc) row_means8(t, e0, mean);
    Ctx cs = c;
    if (c.tflags & APEXW_FLAG_VSCALE) {
      cs.vscale = t.v_scale[0];
      cs.vscale_sqrt = t.v_scale[1];
    }
    // torch's CPU add with alpha over two tensors of one 16-bit dtype (beta3's numerator)
    // rounds alpha to that dtype and computes a + alpha b with one fused multiply-add in its
    // vector loop, 32 elements at a time, but rounds the product to the dtype first in the
    // scalar loop that ends each tensor (its last n % 32 elements); tj: this group's first
    // element in that remainder (8: none)
    int tj = 8;
    if constexpr (VAR && !QUAD) {
      const int64_t rel = (t.n - (t.n & 31)) - e0;
      tj = rel < 0 ? 0 : (rel > 8 ? 8 : (int)rel);
    }
    update8<PD, GD, MD, VD, QUAD, SR, VAR>(p, g, m, v, x, ms, cnt, (uint32_t)e0, cs, gc, mean, ams, slow, tj);
    if (full) {
      store8<PD>(t.p, e0, p);
      store8<MD>(t.m, e0, m);
      if (slow) store8<MD>(mslow, e0, ms);
      if constexpr (QUAD) {
        if constexpr (VD == APEXW_F32) {
          u32x2 w = {__float_as_uint(v[0]), __float_as_uint(v[1])};
          __builtin_nontemporal_store(w, (u32x2*)((float*)t.v + (e0 >> 2)));
        } else {
          const uint32_t lo = VD == APEXW_BF16 ? (__float_as_uint(v[0]) >> 16) : f32_to_f16_bits(v[0]);
          const uint32_t hi = VD == APEXW_BF16 ? (__float_as_uint(v[1]) >> 16) : f32_to_f16_bits(v[1]);
          __builtin_nontemporal_store(lo | (hi << 16), (uint32_t*)((uint16_t*)t.v + (e0 >> 2)));
        }
      } else if (!lion) {
        store8<VD>(t.v, e0, v);
        if (ams) store8<VD>(vmax, e0, x);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j < cnt) {
          store1<PD>(t.p, e0 + j, p[j]);
          store1<MD>(t.m, e0 + j, m[j]);
          if constexpr (!QUAD) {
            if (!lion) store1<VD>(t.v, e0 + j, v[j]);
          }
          if (ams) store1<VD>(vmax, e0 + j, x[j]);
          if (slow) store1<MD>(mslow, e0 + j, ms[j]);
        }
      }
      if constexpr (QUAD) {
        if (cnt >= 4) store1<VD>(t.v, e0 >> 2, v[0]);
        if (cnt >= 8) store1<VD>(t.v, (e0 >> 2) + 1, v[1]);
      }
    }
  }
}

// The grad dtype of a group: the parameter's in the plain instantiation; any of the
// three in the variant one (APEXW_HP_GRAD_DTYPES launches)
template <int PD, int MD, int VD, bool QUAD, bool SR, bool VAR>
APEXW_DEV void group_gd(const apexw_tensor& t, int64_t start, int k, const Ctx& c, void* vmax, void* mslow,
                        uint32_t gd) {
  if constexpr (VAR) {
    if (gd != (uint32_t)PD) {
      if (gd == APEXW_F32) compact_group<PD, APEXW_F32, MD, VD, QUAD, SR, VAR>(t, start, k, c, vmax, mslow);
      else if (gd == APEXW_BF16) compact_group<PD, APEXW_BF16, MD, VD, QUAD, SR, VAR>(t, start, k, c, vmax, mslow);
      else compact_group<PD, APEXW_F16, MD, VD, QUAD, SR, VAR>(t, start, k, c, vmax, mslow);
      return;
    }
  }
  compact_group<PD, PD, MD, VD, QUAD, SR, VAR>(t, start, k, c, vmax, mslow);
}

template <bool SR, bool VAR>
APEXW_DEV void dispatch_group(const apexw_tensor& t, int64_t start, int k, const Ctx& c, uint32_t pd, uint32_t md,
                              uint32_t vd, bool quad, void* vmax, void* mslow, uint32_t gd) {
  if (md == APEXW_F32) {
    // fp32 moments ("full" precision, small "auto" tensors): fp32 v, no quad (checked on the host)
    if (pd == APEXW_F32) group_gd<APEXW_F32, APEXW_F32, APEXW_F32, false, SR, VAR>(t, start, k, c, vmax, mslow, gd);
    else if (pd == APEXW_BF16) group_gd<APEXW_BF16, APEXW_F32, APEXW_F32, false, SR, VAR>(t, start, k, c, vmax, mslow, gd);
    else group_gd<APEXW_F16, APEXW_F32, APEXW_F32, false, SR, VAR>(t, start, k, c, vmax, mslow, gd);
    return;
  }
  if (pd == APEXW_F16) {
    // fp16 parameters keep fp16 m (and fp16 or fp32 v)
    if (vd == APEXW_F32) group_gd<APEXW_F16, APEXW_F16, APEXW_F32, false, SR, VAR>(t, start, k, c, vmax, mslow, gd);
    else if (quad) group_gd<APEXW_F16, APEXW_F16, APEXW_F16, true, SR, VAR>(t, start, k, c, vmax, mslow, gd);
    else group_gd<APEXW_F16, APEXW_F16, APEXW_F16, false, SR, VAR>(t, start, k, c, vmax, mslow, gd);
    return;
  }
  if (pd == APEXW_F32) {
    if (vd == APEXW_F32) group_gd<APEXW_F32, APEXW_BF16, APEXW_F32, false, SR, VAR>(t, start, k, c, vmax, mslow, gd);
    else if (quad) group_gd<APEXW_F32, APEXW_BF16, APEXW_BF16, true, SR, VAR>(t, start, k, c, vmax, mslow, gd);
    else group_gd<APEXW_F32, APEXW_BF16, APEXW_BF16, false, SR, VAR>(t, start, k, c, vmax, mslow, gd);
  } else {
    if (vd == APEXW_F32) group_gd<APEXW_BF16, APEXW_BF16, APEXW_F32, false, SR, VAR>(t, start, k, c, vmax, mslow, gd);
    else if (quad) group_gd<APEXW_BF16, APEXW_BF16, APEXW_BF16, true, SR, VAR>(t, start, k, c, vmax, mslow, gd);
    else group_gd<APEXW_BF16, APEXW_BF16, APEXW_BF16, false, SR, VAR>(t, start, k, c, vmax, mslow, gd);
  }
}

// cautious count pass: of group k (8 elements per lane) of the unit at `start`, the
// elements whose mask is set, from the grads as the step prepares them and the first
// moment as it updates it (nothing is written)
template <int PD, int GD, int MD, bool QUAD>
APEXW_DEV uint32_t count_group(const apexw_tensor& t, int64_t start, int k, const Ctx& c) {
  const int64_t e0 = start + (int64_t)(k * 64 + lane_id()) * 8;
  if (e0 >= t.n) return 0u;
  const int cnt = (int)((t.n - e0) < 8 ? (t.n - e0) : 8);
  float g[8], m[8];
  if (!(c.tflags & APEXW_FLAG_SCALAR) && cnt == 8) {
    load8<GD>(t.g, e0, g);
    load8<MD>(t.m, e0, m);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      g[j] = j < cnt ? load1<GD>(t.g, e0 + j) : 0.0f;
      m[j] = j < cnt ? load1<MD>(t.m, e0 + j) : 0.0f;
    }
  }
  const bool gc = c.tflags & APEXW_FLAG_GC;
  float mean[8];
  if (gc) row_means8(t, e0, mean);
  const bool san = (c.hp->flags & APEXW_HP_SANITIZE) && any_nonfinite8(g);
#pragma unroll
  for (int j = 0; j < 8; ++j) g[j] = prep_grad<GD>(g[j], c, san, gc, mean[j]);
  m_update8<GD, MD>(m, g, *c.hp);
  uint32_t n_set = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) n_set += (j < cnt && caut_mask<GD, QUAD>(g[j], m[j], c.hp->mode)) ? 1u : 0u;
  return n_set;
}

template <int PD, int MD, bool QUAD>
APEXW_DEV uint32_t count_gd(const apexw_tensor& t, int64_t start, int k, const Ctx& c, uint32_t gd) {
  if (gd == APEXW_F32) return count_group<PD, APEXW_F32, MD, QUAD>(t, start, k, c);
  if (gd == APEXW_BF16) return count_group<PD, APEXW_BF16, MD, QUAD>(t, start, k, c);
  return count_group<PD, APEXW_F16, MD, QUAD>(t, start, k, c);
}

APEXW_DEV uint32_t dispatch_count(const apexw_tensor& t, int64_t start, int k, const Ctx& c, uint32_t pd, uint32_t md,
                                  bool quad, uint32_t gd) {
  if (md == APEXW_F32) {
    if (pd == APEXW_F32) return count_gd<APEXW_F32, APEXW_F32, false>(t, start, k, c, gd);
    if (pd == APEXW_BF16) return count_gd<APEXW_BF16, APEXW_F32, false>(t, start, k, c, gd);
    return count_gd<APEXW_F16, APEXW_F32, false>(t, start, k, c, gd);
  }
  if (pd == APEXW_F16)
    return quad ? count_gd<APEXW_F16, APEXW_F16, true>(t, start, k, c, gd)
                : count_gd<APEXW_F16, APEXW_F16, false>(t, start, k, c, gd);
  if (pd == APEXW_F32)
    return quad ? count_gd<APEXW_F32, APEXW_BF16, true>(t, start, k, c, gd)
                : count_gd<APEXW_F32, APEXW_BF16, false>(t, start, k, c, gd);
  return quad ? count_gd<APEXW_BF16, APEXW_BF16, true>(t, start, k, c, gd)
              : count_gd<APEXW_BF16, APEXW_BF16, false>(t, start, k, c, gd);
}

// Per tensor, the count of set mask bits into hp.counts (cleared before the pass);
// the work items are the step kernel's.
__global__ __launch_bounds__(256) void compact_count_kernel(const apexw_tensor* __restrict__ tensors,
                                                            const apexw_unit* __restrict__ units,
                                                            int64_t n_units, apexw_hparams hp_in) {
  apexw_hparams hp = hp_in;
  if (hp.flags & APEXW_HP_AMP) {
    const apexw_amp_dyn d = *hp.amp;
    if (d.skip) return;
    hp.grad_inv_scale = d.grad_inv_scale;
  }
  const uint32_t wave = uniform(threadIdx.x >> 6);
  Ctx c;
  c.hp = &hp;
  c.coef = (hp.flags & APEXW_HP_CLIP) ? *hp.clip_coef : 1.0f;
  c.vscale = c.vscale_sqrt = 1.0f;
  c.cq = 0.0f;
  const int64_t n_items = n_units * kGroups;
  for (int64_t w = (int64_t)blockIdx.x * kWaves + wave; w < n_items; w += (int64_t)gridDim.x * kWaves) {
    const apexw_unit un = units[w / kGroups];
    const apexw_tensor& t = tensors[un.tensor];
    if (t.flags & APEXW_FLAG_FACTORED) continue;
    c.tflags = t.flags;
    const uint32_t pd = (t.flags >> APEXW_FLAG_PDT_SHIFT) & 3u, md = (t.flags >> APEXW_FLAG_MDT_SHIFT) & 3u;
    uint32_t n_set = dispatch_count(t, (int64_t)un.unit * APEXW_COMPACT_UNIT, (int)(w % kGroups), c, pd, md,
                                    t.flags & APEXW_FLAG_QUAD, (t.flags >> APEXW_FLAG_GDT_SHIFT) & 3u);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) n_set += __shfl_xor(n_set, off, 64);
    if (lane_id() == 0 && n_set) atomicAdd(&hp.counts[un.tensor], (unsigned long long)n_set);
  }
}

__global__ __launch_bounds__(256) void compact_counts_zero_kernel(unsigned long long* __restrict__ counts,
                                                                  int32_t n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) counts[i] = 0ull;
}

template <bool VAR>
__global__ __launch_bounds__(256) void compact_step_kernel(const apexw_tensor* __restrict__ tensors,
                                                           const apexw_unit* __restrict__ units,
                                                           int64_t n_units, apexw_hparams hp_in) {
  apexw_hparams hp = hp_in;
  if (hp.flags & APEXW_HP_AMP) {
    // GradScaler's step read on the device: skip it (found_inf) or take its scalars
    const apexw_amp_dyn d = *hp.amp;
    if (d.skip) return;
    hp.step_size = d.step_size;
    hp.eps_scaled = d.eps_scaled;
    hp.bc2_sqrt = d.bc2_sqrt;
    hp.grad_inv_scale = d.grad_inv_scale;
  }
  const uint32_t wave = uniform(threadIdx.x >> 6);
  Ctx c;
  c.hp = &hp;
  c.coef = (hp.flags & APEXW_HP_CLIP) ? *hp.clip_coef : 1.0f;
  c.vscale = 1.0f;
  c.vscale_sqrt = 1.0f;
  c.cq = 0.0f;
  // SR applies to the 16-bit stores of the cold and replayed steps (the native and
  // per-parameter modes never set it)
  const bool sr = (hp.flags & APEXW_HP_SR) && (hp.mode == APEXW_MODE_COLD || hp.mode == APEXW_MODE_REPLAY);
  // one work item = one 512-element group of a unit, so a small launch still
  // puts four waves per unit in flight (the per-element RNG is keyed by the
  // element index, so the split does not change any result)
  // workgroup b takes items [chunk b, chunk (b + 1)), then strides by the grid (a
  // grid of one workgroup per unit makes that one pass, see apexw_launch_compact)
  const int64_t n_items = n_units * kGroups;
  for (int64_t base = (int64_t)blockIdx.x * kWaves; base < n_items; base += (int64_t)gridDim.x * kWaves)
  for (int64_t w = base + wave; w < base + kWaves && w < n_items; w += kWaves) {
    const apexw_unit un = units[w / kGroups];
    const int k = (int)(w % kGroups);
    const apexw_tensor& t = tensors[un.tensor];
    const int64_t start = (int64_t)un.unit * APEXW_COMPACT_UNIT;
    c.tflags = t.flags;
    c.key = rng_key(hp.seed, un.tensor, hp.step, 0u, (uint32_t)(start >> 32));
    const uint32_t pd = (t.flags >> APEXW_FLAG_PDT_SHIFT) & 3u;
    const uint32_t md = (t.flags >> APEXW_FLAG_MDT_SHIFT) & 3u;
    const uint32_t vd = (t.flags >> APEXW_FLAG_VDT_SHIFT) & 3u;
    const bool quad = t.flags & APEXW_FLAG_QUAD;
    const uint32_t gd = (t.flags >> APEXW_FLAG_GDT_SHIFT) & 3u;
    if (quad && hp.mode == APEXW_MODE_SINGLE) continue;  // rejected on the host; never read v out of range
    // a grad of another dtype than its parameter: only the variant instantiation reads it
    // (APEXW_HP_GRAD_DTYPES); the plain one never reads a grad at the wrong width
    if (!VAR && gd != pd) continue;
    if (t.flags & APEXW_FLAG_FACTORED) continue;        // stepped by apexw_factored_step
    if (VAR && (hp.flags & APEXW_HP_CAUTIOUS)) c.cq = caut_q(hp.counts[un.tensor], t.n, quad, pd);
    void* vmax = (VAR && (hp.flags & APEXW_HP_AMSGRAD) && !quad) ? hp.max_v[un.tensor] : nullptr;
    void* mslow = (VAR && (hp.flags & APEXW_HP_SLOW) && !quad) ? hp.slow[un.tensor] : nullptr;
    if (sr) dispatch_group<true, VAR>(t, start, k, c, pd, md, vd, quad, vmax, mslow, gd);
    else dispatch_group<false, VAR>(t, start, k, c, pd, md, vd, quad, vmax, mslow, gd);
  }
}

}  // namespace

// Host-side validation of the dtype combinations this kernel instantiates.
static bool compact_combo_ok(uint32_t flags) {
  const uint32_t pd = (flags >> APEXW_FLAG_PDT_SHIFT) & 3u, gd = (flags >> APEXW_FLAG_GDT_SHIFT) & 3u;
  const uint32_t md = (flags >> APEXW_FLAG_MDT_SHIFT) & 3u, vd = (flags >> APEXW_FLAG_VDT_SHIFT) & 3u;
  // the grads may be of another dtype than their parameter (read by the variant instantiation)
  if (!(pd == APEXW_F32 || pd == APEXW_BF16 || pd == APEXW_F16) || !(gd == APEXW_F32 || gd == APEXW_BF16 || gd == APEXW_F16))
    return false;
  if (md == APEXW_F32) return vd == APEXW_F32 && !(flags & APEXW_FLAG_QUAD);   // fp32 moments
  // 16-bit moments are in the parameter's compact dtype: fp16 for fp16, else bf16
  const uint32_t cd = pd == APEXW_F16 ? APEXW_F16 : APEXW_BF16;
  if (md != cd || !(vd == APEXW_F32 || vd == cd)) return false;
  if ((flags & APEXW_FLAG_QUAD) && vd != cd) return false;
  return true;
}

int apexw_launch_compact(const apexw_tensor* tensors, int64_t n_units, const apexw_unit* units,
                         const apexw_hparams* hp, hipStream_t stream) {
  // Large launches: one workgroup per unit (its four 512-element groups, one per
  // wave), so the resident workgroups sweep a narrow, advancing window of the
  // tensors (C4, 2.16 B elements: 5.45-5.51 ms per step against 5.75-5.95 with a
  // resident grid striding over the whole launch).  Launches that a resident grid
  // covers in a few passes keep it (C2, 124 M elements: 0.234-0.257 ms against
  // 0.252-0.288 with a workgroup per unit).
  // nesterov / cautious / amsgrad / lion / beta3 launches, and those with grads of another dtype
  // than their parameters, take the instantiation that holds them
  const bool var = hp->flags & (APEXW_HP_NESTEROV | APEXW_HP_CAUTIOUS | APEXW_HP_AMSGRAD | APEXW_HP_LION |
                                APEXW_HP_SLOW | APEXW_HP_GRAD_DTYPES);
  const void* kernel = var ? (const void*)compact_step_kernel<true> : (const void*)compact_step_kernel<false>;
  const int resident = apexw_resident_grid(kernel, n_units * kGroups);
  const int grid = n_units > (int64_t)resident * 8 ? (int)(n_units < INT32_MAX ? n_units : INT32_MAX) : resident;
  if (var)
    hipLaunchKernelGGL(compact_step_kernel<true>, dim3(grid), dim3(256), 0, stream, tensors, units, n_units, *hp);
  else
    hipLaunchKernelGGL(compact_step_kernel<false>, dim3(grid), dim3(256), 0, stream, tensors, units, n_units, *hp);
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

int apexw_launch_compact_cautious_count(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units,
                                        int64_t n_units, const apexw_hparams* hp, hipStream_t stream) {
  // the counters are cleared by a kernel (not hipMemsetAsync), which a captured graph replays reliably
  hipLaunchKernelGGL(compact_counts_zero_kernel, dim3((unsigned)((n_tensors + 255) / 256)), dim3(256), 0, stream,
                     hp->counts, n_tensors);
  if (n_units > 0) {
    const int grid = apexw_resident_grid((const void*)compact_count_kernel, n_units * kGroups);
    hipLaunchKernelGGL(compact_count_kernel, dim3(grid), dim3(256), 0, stream, tensors, units, n_units, *hp);
  }
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

bool apexw_compact_flags_ok(uint32_t flags) { return compact_combo_ok(flags); }
