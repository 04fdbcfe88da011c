// 8-bit fused multi-tensor AdamW step (gfx950).
//
// One wavefront owns one quantization block (<= 2048 elements, 32 per lane in 4
// groups of 8 consecutive elements one wave-width apart).  A block is
// dequantized, updated and requantized entirely in registers: the absmax of the
// new momentum and the max of the new variance are wavefront reductions, so no
// LDS round trip or barrier is needed between the update and the requantization.
// LDS only holds the decode tables (256-entry log-uint8 LUT, NF4 codebook),
// loaded once per persistent workgroup.
//
// Arithmetic restates the reference's CPU 8-bit path ApexW._step_ultra
// (apexw/optimizer.py:4313-4735): chunked order for large tensors (:4402-4499),
// generic order for other quantized tensors (:4538-4639), and the 16-bit state
// fallback for tensors under 64 elements (:4688-4735).  Quantizers follow
// apexw/quantization.py (INT8 :66-126, NF4 :277-357, log-uint8 :381-448).
#include "common.h"
#include "luts.h"

// A tensor takes the full-block kernel when it has bf16 params/grads, NF4 m,
// quad log-uint8 v, 2048-element blocks and 16-byte aligned buffers.
static __host__ __device__ inline bool apexw_q8_fast_ok(uint32_t flags, uint32_t block) {
  const uint32_t pd = (flags >> APEXW_FLAG_PDT_SHIFT) & 3u, gd = (flags >> APEXW_FLAG_GDT_SHIFT) & 3u;
  return (pd == APEXW_BF16 || pd == APEXW_F32) && gd == pd && (flags & APEXW_FLAG_NF4) &&
         (flags & APEXW_FLAG_QUAD) && !(flags & (APEXW_FLAG_SCALAR | APEXW_FLAG_DENSE | APEXW_FLAG_FACTORED)) &&
         block == 2048;
}

namespace {

constexpr int kWaves = 4;
// units per workgroup of the full-block kernels: a small chunk keeps the resident
// workgroups on a narrow, advancing window of the tensors; 4 is one unit per wave
// (C3, 8.03 B parameters, one box: 10.76 ms per step with 4 units, 10.91 with 8,
// 11.39 with 16; on an earlier build 8 -> 64 units went 11.27 -> 11.67 ms)
constexpr int64_t kFastChunk = 4;

struct Q8Ctx {
  const apexw_hparams* hp;
  const float* vlut;   // LDS: log-uint8 decode table
  const float* code;   // LDS: NF4 codebook
  const float2* pair;    // LDS: NF4 byte -> two values
  const float4* frac16;  // LDS: signed fractional NF4 code buckets (x 4096, +7, lines in y = x + 3)
  const float2* midtab;  // LDS: NF4 round-to-nearest buckets (kNf4MidTab)
  float coef;
  // grad centralization of the current unit's tensor (APEXW_FLAG_GC): its fp32 row
  // means and row length from the launch's side table (hparams.rows), else nullptr
  const float* gc_means;
  int64_t gc_rl;
  // the SNR gains of the current unit's tensor: the launch's, or with cautious=True
  // (q_t, 0), q_t = 1 / max(c_t / n_t, 1e-3) from the tensor's mask count
  float gain_hi, gain_lo;
};

// The gains of tensor tix (APEXW_HP_CAUTIOUS: the cautious mask's 1 / mean and 0;
// torch's float32 mean of the 0 / 1 mask is the count over n, exactly rounded,
// for tensors of up to 2^24 elements, apexw/optimizer.py:4585-4588).
APEXW_DEV void q8_set_gains(Q8Ctx& c, const apexw_tensor& t, uint32_t tix) {
  const apexw_hparams& hp = *c.hp;
  if (hp.flags & APEXW_HP_CAUTIOUS) {
    const float mean = fmaxf((float)hp.counts[tix] / (float)t.n, 1e-3f);
    c.gain_hi = 1.0f / mean;
    c.gain_lo = 0.0f;
  } else {
    c.gain_hi = hp.gain_hi;
    c.gain_lo = hp.gain_lo;
  }
}

// Point the context at the row means of tensor tix (or at none).
APEXW_DEV void q8_set_rows(Q8Ctx& c, const apexw_tensor& t, uint32_t tix) {
  c.gc_means = nullptr;
  c.gc_rl = 0;
  if ((t.flags & APEXW_FLAG_GC) && c.hp->rows) {
    const apexw_row_means r = c.hp->rows[tix];
    c.gc_means = r.means;
    c.gc_rl = r.row_len;
  }
}

// a / b for 0 <= a, 0 < b, in 32 bits when both fit (a 64-bit division is a long
// software sequence)
APEXW_DEV int64_t q8_udiv(int64_t a, int64_t b) {
  if (((uint64_t)a | (uint64_t)b) >> 32) return a / b;
  return (int64_t)((uint32_t)a / (uint32_t)b);
}

// Row means of the 8 elements from e0 of a centralized tensor; zeros otherwise.
APEXW_DEV void q8_means8(const Q8Ctx& c, const apexw_tensor& t, int64_t e0, float (&mean)[8]) {
  if (!c.gc_means) {
#pragma unroll
    for (int j = 0; j < 8; ++j) mean[j] = 0.0f;
    return;
  }
  const int64_t rl = c.gc_rl, rows = q8_udiv(t.n, rl);
  if (rl >= 8) {
    // at most one row boundary inside the 8 elements
    const int64_t row = q8_udiv(e0, rl), col = e0 - row * rl;
    const float m0 = c.gc_means[row < rows ? row : rows - 1];
    const float m1 = (col + 8 > rl && row + 1 < rows) ? c.gc_means[row + 1] : m0;
#pragma unroll
    for (int j = 0; j < 8; ++j) mean[j] = col + j < rl ? m0 : m1;
    return;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t r = q8_udiv(e0 + j, rl);
    mean[j] = c.gc_means[r < rows ? r : rows - 1];
  }
}

APEXW_DEV float q8_mean1(const Q8Ctx& c, const apexw_tensor& t, int64_t i) {
  if (!c.gc_means) return 0.0f;
  const int64_t r = q8_udiv(i, c.gc_rl), rows = q8_udiv(t.n, c.gc_rl);
  return c.gc_means[r < rows ? r : rows - 1];
}

// The row means of one 2048-element block of a centralized tensor whose rows hold
// at least 2048 elements: the block meets at most one row boundary, so elements
// below `split` take m0 and the others m1 (one division per block, not per element).
struct BlockMeans {
  int64_t split;
  float m0, m1;
  bool one;    // rows of >= 2048 elements: split / m0 / m1 hold
  bool by8;    // and of a multiple of 8 elements: no 8-element group straddles two rows
};

APEXW_DEV BlockMeans q8_block_means(const Q8Ctx& c, const apexw_tensor& t, int64_t start) {
  BlockMeans b{0, 0.0f, 0.0f, false, false};
  if (!c.gc_means || c.gc_rl < 2048) return b;
  const int64_t rl = c.gc_rl, rows = q8_udiv(t.n, rl);
  const int64_t row = q8_udiv(start, rl);
  b.one = true;
  b.by8 = (rl & 7) == 0;
  b.split = (row + 1) * rl;
  b.m0 = c.gc_means[row < rows ? row : rows - 1];
  b.m1 = row + 1 < rows ? c.gc_means[row + 1] : b.m0;
  return b;
}

// Division by a denominator shared across a quad or a block, round-to-nearest:
// r = RN-refined 1/y (one Newton step on v_rcp_f32), q0 = x r, then the exact
// FMA residual e = x - q0 y corrects q0 (Markstein): the result equals the IEEE
// quotient except within ~2^-46 of a rounding midpoint.  y is positive, finite
// and normal at every call site (scales >= 1e-12, denominators >= eps).
APEXW_DEV float rcp_refined(float y) {
  const float r0 = __builtin_amdgcn_rcpf(y);
  return fmaf(fmaf(-y, r0, 1.0f), r0, r0);
}
APEXW_DEV float div_shared(float x, float y, float r) {
  const float q0 = x * r;
  return fmaf(fmaf(-q0, y, x), r, q0);
}

APEXW_DEV float lerp_to(float a, float b, float coef, bool hi) {
  // torch lerp(a, b, w): |w| < 0.5 -> a + w*(b-a); else b + (w-1)*(b-a), one FMA each
  return hi ? fmaf(coef, b - a, b) : fmaf(coef, b - a, a);
}

// NF4 nearest code, searchsorted(mids, x) over the 14 decision points (ties to the
// lower code), through the 64-bucket midpoint table (LDS copy of kNf4MidTab):
// one lookup and one comparison.
APEXW_DEV uint32_t nf4_rne_tab(float x, const float2* tab) {
  const float a = fabsf(x);
  const float2 e = tab[min((int)(a * 64.0f), 63)];
  const uint32_t base = (uint32_t)e.x;
  return x >= 0.0f ? 7u + base + (e.y < a ? 1u : 0u) : 7u - base - (e.y <= a ? 1u : 0u);
}

// NF4 stochastic code: hi = #(levels[0..14] < x), lo = hi - 1, P(hi) = (x - c_lo)/(c_hi - c_lo).
APEXW_DEV uint32_t nf4_sr(float x, float u, const float* code) {
  uint32_t hi = 0;
#pragma unroll
  for (int k = 0; k < 15; ++k) hi += (code[k] < x) ? 1u : 0u;
  hi = hi > 14u ? 14u : hi;
  const uint32_t lo = hi > 0u ? hi - 1u : 0u;
  const float c_lo = code[lo], c_hi = code[hi];
  const float gap = c_hi - c_lo;
  const float p_hi = gap > 0.0f ? (x - c_lo) / fmaxf(gap, 1e-12f) : 1.0f;
  return u < p_hi ? hi : lo;
}

APEXW_DEV float unit_uniform(uint32_t r16) { return ((float)(r16 & 0xFFFFu) + 0.5f) * (1.0f / 65536.0f); }

// log-uint8 code of v given the block scale (ratio floor 2^-24, 254 codes per 24 octaves).
APEXW_DEV uint32_t logu8_code(float v, float vmax, bool sr, uint32_t r16) {
  if (!(v > 0.0f)) return 0u;
  const float r = fmaxf(v / vmax, 0x1p-24f);
  float q = log2f(r) * 0x1.52aaaap+3f;  // fp32(254/24)
  q = q + 255.0f;
  if (sr) q = q + (unit_uniform(r16) - 0.5f);
  q = rintf(q);
  q = fminf(fmaxf(q, 1.0f), 255.0f);
  return (uint32_t)q;
}

// logu8_code (round to nearest) with the block's shared reciprocal for v / vmax
APEXW_DEV uint32_t logu8_code_shared(float v, float vmax, float rvmax) {
  if (!(v > 0.0f)) return 0u;
  const float r = fmaxf(div_shared(v, vmax, rvmax), 0x1p-24f);
  // r >= 2^-24 is a normal number, where log2f is v_log_f32 itself (its scaling of
  // denormal inputs never applies)
  const float q = rintf(__builtin_amdgcn_logf(r) * 0x1.52aaaap+3f + 255.0f);
  return (uint32_t)fminf(fmaxf(q, 1.0f), 255.0f);
}

// nan_to_num inside the step: on the fp32 copy (chunked) or on the grad dtype (generic)
template <int GD> APEXW_DEV float q8_nan_to_num(float g, uint32_t tflags) {
  if (__builtin_isnan(g)) return 0.0f;
  if (__builtin_isinf(g)) {
    const float big = (tflags & (APEXW_FLAG_GENERIC | APEXW_FLAG_DENSE)) ? rnd<GD>(65504.0f) : 65504.0f;
    return g > 0.0f ? big : -big;
  }
  return g;
}

// True when any of the 8 values is NaN or +-Inf (x * 0 is NaN exactly then).
APEXW_DEV bool q8_any_nonfinite8(const float (&x)[8]) {
  float t = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) t = fmaf(x[j], 0.0f, t);
  return !(t == t);
}

// mean: the element's row mean when its tensor is centralized (c.gc_means).
template <int GD> APEXW_DEV float q8_grad(float g, uint32_t tflags, const Q8Ctx& c, float mean = 0.0f) {
  const apexw_hparams& hp = *c.hp;
  const bool unscale = hp.flags & APEXW_HP_UNSCALE, clip = hp.flags & APEXW_HP_CLIP;
  const bool gc = c.gc_means != nullptr;
  if (hp.flags & APEXW_HP_SANITIZE) g = sanitize<GD>(g);
  // AMP before a clip or a centralization: _prepare_grads unscales in the grad dtype
  // (apexw/optimizer.py:227-237), then subtracts each row's mean (:239-243), then clips
  if (unscale && (clip || gc)) g = rnd<GD>(g * hp.grad_inv_scale);
  if (gc) g = rnd<GD>(g - mean);
  if (clip) g = rnd<GD>(g * c.coef);
  g = q8_nan_to_num<GD>(g, tflags);
  // AMP without a clip: the step unscales its fp32 copy after nan_to_num
  // (_prep_grad_chunk_fp32, apexw/state.py:326-347; apexw/optimizer.py:4500-4505)
  if (unscale && !clip && !gc) g *= hp.grad_inv_scale;
  return g;
}

template <int PD>
APEXW_DEV float q8_param(float p, float upd, float decay, uint32_t tflags, bool sr, bool quad, uint32_t r) {
  const bool wd = tflags & APEXW_FLAG_WD;
  if (tflags & APEXW_FLAG_GENERIC) {
    // p.mul_(decay) first, then p -= bf16(update) (SR only for quad-v tensors)
    if (wd) p = rnd<PD>(p * decay);
    if constexpr (PD == APEXW_F32) return p - upd;
    if (quad && sr) return sr_round<PD>(p - upd, r);
    return rnd<PD>(p - rnd<PD>(upd));
  }
  if (wd) p = p * decay;
  if constexpr (PD == APEXW_F32) return p - upd;
  const float x = p - upd;
  if (sr) return sr_round<PD>(x, r);
  // the fp32 -> 16-bit copy (_copy_fp32_to_16bit_sr_) clamps fp16 to its range
  if constexpr (PD == APEXW_F16) return rnd<PD>(clamp_f16_range(x));
  return rnd<PD>(x);
}

// One quantization block per wavefront, any layout (INT8 m, fp32 params, other
// block sizes, unaligned tensors).  Runs in its own kernel so that its register
// footprint does not lower the occupancy of the bf16 NF4 kernel below.
// SINGLE: the per-parameter in-backward update (ApexW._step_single_param_fused,
// apexw/optimizer.py:2411-2457): raw fp32 grads, m = b1 m + (1-b1) g,
// lookahead b1 m' + (1-b1) g, denominator sqrt(v) + eps_scaled without the eps
// floor, p decayed in fp32 then p + (-step_size * num) / den, INT8 m
// requantised from its own absmax (no EMA, no SR).
template <int PD, bool NF4, bool QUAD, bool SINGLE>
APEXW_DEV void q8_block(const apexw_tensor& t, uint32_t tix, uint32_t blk, const Q8Ctx& c) {
  constexpr int GD = PD;
  const apexw_hparams& hp = *c.hp;
  const bool sr = hp.flags & APEXW_HP_SR;
  const uint32_t tflags = t.flags;
  const bool vec = !(tflags & APEXW_FLAG_SCALAR);
  const int64_t bs = t.block;
  const int64_t start = (int64_t)blk * bs;
  const int64_t cnt_blk = (t.n - start) < bs ? (t.n - start) : bs;
  const int lane = lane_id();
  const float ms_old = t.m_scale[blk];
  const float vs_old = t.v_scale[blk];
  const uint32_t key = rng_key(hp.seed, tix, hp.step, 1u, (uint32_t)(start >> 32));
  const uint32_t keyv = rng_key(hp.seed, tix, hp.step, 2u, (uint32_t)(start >> 32));
  const bool generic = tflags & APEXW_FLAG_GENERIC;

  float mnew[4][8], vnew[4][8];
  float amax = 0.0f, vmax = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t rel = (int64_t)(k * 64 + lane) * 8;
    const int cnt = rel >= cnt_blk ? 0 : (int)((cnt_blk - rel) < 8 ? (cnt_blk - rel) : 8);
#pragma unroll
    for (int j = 0; j < 8; ++j) { mnew[k][j] = 0.0f; vnew[k][j] = 0.0f; }
    if (cnt == 0) continue;
    const int64_t e0 = start + rel;
    const bool full = vec && cnt == 8;
    float p[8], g[8], m[8], v[8];
    // ---- load
    if (full) {
      load8<PD>(t.p, e0, p);
      load8<GD>(t.g, e0, g);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        p[j] = j < cnt ? load1<PD>(t.p, e0 + j) : 0.0f;
        g[j] = j < cnt ? load1<GD>(t.g, e0 + j) : 0.0f;
      }
    }
    if constexpr (NF4) {
      uint32_t codes[8];
      if (full) {
        const uint32_t w = __builtin_nontemporal_load((const uint32_t*)((const uint8_t*)t.m + (e0 >> 1)));
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const uint32_t byte = (w >> (8 * b)) & 0xFFu;
          codes[2 * b] = byte >> 4;
          codes[2 * b + 1] = byte & 15u;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t byte = j < cnt ? ((const uint8_t*)t.m)[(e0 + j) >> 1] : 0x77u;
          codes[j] = ((e0 + j) & 1) ? (byte & 15u) : (byte >> 4);
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) m[j] = c.code[codes[j]] * ms_old;
    } else {
      if (full) {
        const u32x2 w = __builtin_nontemporal_load((const u32x2*)((const int8_t*)t.m + e0));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t word = j < 4 ? w.x : w.y;
          m[j] = (float)(int8_t)((word >> (8 * (j & 3))) & 0xFFu) * ms_old;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) m[j] = j < cnt ? (float)((const int8_t*)t.m)[e0 + j] * ms_old : 0.0f;
      }
    }
    if constexpr (QUAD) {
      uint32_t vc[2];
      if (full) {
        const uint32_t w = __builtin_nontemporal_load((const uint16_t*)((const uint8_t*)t.v + (e0 >> 2)));
        vc[0] = w & 0xFFu;
        vc[1] = (w >> 8) & 0xFFu;
      } else {
        vc[0] = cnt >= 4 ? ((const uint8_t*)t.v)[e0 >> 2] : 0u;
        vc[1] = cnt >= 8 ? ((const uint8_t*)t.v)[(e0 >> 2) + 1] : 0u;
      }
      v[0] = c.vlut[vc[0]] * vs_old;
      v[1] = c.vlut[vc[1]] * vs_old;
    } else {
      if (full) {
        const u32x2 w = __builtin_nontemporal_load((const u32x2*)((const uint8_t*)t.v + e0));
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = c.vlut[((j < 4 ? w.x : w.y) >> (8 * (j & 3))) & 0xFFu] * vs_old;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = j < cnt ? c.vlut[((const uint8_t*)t.v)[e0 + j]] * vs_old : 0.0f;
      }
    }
    // ---- update
    uint32_t h[8];
    float mean[8];
    q8_means8(c, t, e0, mean);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      h[j] = sr ? rng_at(key, (uint32_t)(e0 + j)) : 0u;
      if constexpr (SINGLE) {
        m[j] = fmaf(hp.one_minus_beta1, g[j], m[j] * hp.beta1);
      } else {
        g[j] = q8_grad<GD>(g[j], tflags, c, mean[j]);
        m[j] = lerp_to(m[j], g[j], hp.lerp_coef, hp.flags & APEXW_HP_LERP_HI);
      }
    }
    float num[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float look = SINGLE ? fmaf(hp.one_minus_beta1, g[j], m[j] * hp.beta1)
                                : lerp_to(g[j], m[j], hp.look_coef, hp.flags & APEXW_HP_LOOK_HI);
      num[j] = look * ((m[j] * g[j] >= 0.0f) ? c.gain_hi : c.gain_lo);
    }
    float dens[8] = {1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f};  // SINGLE: denominators
    float upd[8];
    if constexpr (QUAD) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (4 * q >= cnt) break;
        const int b = 4 * q;
        float s = g[b] * g[b];
        s = s + g[b + 1] * g[b + 1];
        s = s + g[b + 2] * g[b + 2];
        s = s + g[b + 3] * g[b + 3];
        float vq = fmaf(hp.one_minus_beta2, s * 0.25f, v[q] * hp.beta2);
        if constexpr (SINGLE) {
          // the update sees v as computed; the quantizer's nan_to_num only affects the stored codes
          const float den = sqrtf(vq) + hp.eps_scaled;
#pragma unroll
          for (int i = 0; i < 4; ++i) dens[b + i] = den;
        }
        if (!(fabsf(vq) <= 3.402823466e38f)) vq = 0.0f;  // nan_to_num(0, 0, 0)
        v[q] = vq;
        const float den = fmaxf(sqrtf(vq) + hp.eps_scaled, hp.eps);
#pragma unroll
        for (int i = 0; i < 4; ++i) upd[b + i] = (num[b + i] / den) * hp.step_size;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float vf = fmaf(hp.one_minus_beta2 * g[j], g[j], v[j] * hp.beta2);
        if constexpr (SINGLE) dens[j] = sqrtf(vf) + hp.eps_scaled;
        if (!(fabsf(vf) <= 3.402823466e38f)) vf = 0.0f;
        v[j] = vf;
        const float den = fmaxf(sqrtf(vf) + hp.eps_scaled, hp.eps);
        upd[j] = (num[j] / den) * hp.step_size;
      }
    }
    if constexpr (SINGLE) {
      // p.mul_(wd) (fp32, on a float copy for 16-bit p), p.addcdiv_(num, den, -step_size),
      // then SR or round-to-nearest into a 16-bit parameter
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float pp = (tflags & APEXW_FLAG_WD) ? p[j] * hp.wd_factor : p[j];
        const float x = pp + (-hp.step_size * num[j]) / dens[j];
        if constexpr (PD == APEXW_F32) p[j] = x;
        else p[j] = sr ? sr_round<PD>(x, h[j]) : rnd<PD>(x);
      }
    } else if constexpr (PD == APEXW_F32) {
      if (generic) {
        // p.mul_(decay); p.addcdiv_(num, den, value=-step_size)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float pp = (tflags & APEXW_FLAG_WD) ? p[j] * hp.wd_factor : p[j];
          const float den = QUAD ? fmaxf(sqrtf(v[j >> 2]) + hp.eps_scaled, hp.eps)
                                 : fmaxf(sqrtf(v[j]) + hp.eps_scaled, hp.eps);
          p[j] = pp + (-hp.step_size * num[j]) / den;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = q8_param<PD>(p[j], upd[j], hp.wd_factor, tflags, sr, QUAD, h[j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) p[j] = q8_param<PD>(p[j], upd[j], hp.wd_factor, tflags, sr, QUAD, h[j]);
    }
    if (full) {
      store8<PD>(t.p, e0, p);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < cnt) store1<PD>(t.p, e0 + j, p[j]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < cnt) {
        mnew[k][j] = m[j];
        amax = fmaxf(amax, fabsf(m[j]));
      }
    }
    if constexpr (QUAD) {
      vnew[k][0] = v[0];
      vnew[k][1] = cnt >= 8 ? v[1] : 0.0f;
      vmax = fmaxf(vmax, fmaxf(vnew[k][0], vnew[k][1]));
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j < cnt) {
          vnew[k][j] = v[j];
          vmax = fmaxf(vmax, v[j]);
        }
      }
    }
  }
  // ---- block scales (EMA-max smoothing against the previous scales)
  amax = wave_max(amax);
  vmax = wave_max(vmax);
  float ms = fmaxf(amax, 1e-12f);
  if (!NF4) ms = ms / 127.0f;
  if (NF4 || !SINGLE) ms = fmaxf(ms, ms_old * 0.9f);
  float vs = fmaxf(vmax, 1e-12f);
  vs = fmaxf(vs, vs_old * 0.95f);
  if (lane == 0) {
    t.m_scale[blk] = ms;
    t.v_scale[blk] = vs;
  }
  // ---- requantize
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t rel = (int64_t)(k * 64 + lane) * 8;
    const int cnt = rel >= cnt_blk ? 0 : (int)((cnt_blk - rel) < 8 ? (cnt_blk - rel) : 8);
    if (cnt == 0) continue;
    const int64_t e0 = start + rel;
    const bool full = vec && cnt == 8;
    uint32_t mc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t r = sr ? (rng_at(key, (uint32_t)(e0 + j)) >> 16) : 0u;
      if constexpr (NF4) {
        const float x = fminf(fmaxf(mnew[k][j] / ms, -1.0f), 1.0f);
        mc[j] = sr ? nf4_sr(x, unit_uniform(r), c.code) : nf4_rne_tab(x, c.midtab);
      } else {
        float y = mnew[k][j] / ms;
        if (sr && !SINGLE) y = y + (unit_uniform(r) - 0.5f);
        y = fminf(fmaxf(rintf(y), -127.0f), 127.0f);
        mc[j] = (uint32_t)(int32_t)y & 0xFFu;
      }
    }
    if constexpr (NF4) {
      if (full) {
        uint32_t w = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) w |= ((mc[2 * b] << 4) | mc[2 * b + 1]) << (8 * b);
        __builtin_nontemporal_store(w, (uint32_t*)((uint8_t*)t.m + (e0 >> 1)));
      } else {
        // element pairs (2i, 2i+1) share a byte; e0 is even, odd tails pad with code 7
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          if (j < cnt) {
            const uint32_t lo = (j + 1 < cnt) ? mc[j + 1] : 7u;
            ((uint8_t*)t.m)[(e0 + j) >> 1] = (uint8_t)((mc[j] << 4) | lo);
          }
        }
      }
    } else {
      if (full) {
        u32x2 w = {mc[0] | (mc[1] << 8) | (mc[2] << 16) | (mc[3] << 24),
                   mc[4] | (mc[5] << 8) | (mc[6] << 16) | (mc[7] << 24)};
        __builtin_nontemporal_store(w, (u32x2*)((int8_t*)t.m + e0));
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (j < cnt) ((uint8_t*)t.m)[e0 + j] = (uint8_t)mc[j];
      }
    }
    if constexpr (QUAD) {
      uint32_t vc[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t r = sr ? rng_at(keyv, (uint32_t)((e0 >> 2) + q)) : 0u;
        vc[q] = logu8_code(vnew[k][q], vs, sr, r);
      }
      if (full) {
        __builtin_nontemporal_store((uint16_t)(vc[0] | (vc[1] << 8)), (uint16_t*)((uint8_t*)t.v + (e0 >> 2)));
      } else {
        if (cnt >= 4) ((uint8_t*)t.v)[e0 >> 2] = (uint8_t)vc[0];
        if (cnt >= 8) ((uint8_t*)t.v)[(e0 >> 2) + 1] = (uint8_t)vc[1];
      }
    } else {
      uint32_t vc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t r = sr ? rng_at(keyv, (uint32_t)(e0 + j)) : 0u;
        vc[j] = logu8_code(vnew[k][j], vs, sr, r);
      }
      if (full) {
        u32x2 w = {vc[0] | (vc[1] << 8) | (vc[2] << 16) | (vc[3] << 24),
                   vc[4] | (vc[5] << 8) | (vc[6] << 16) | (vc[7] << 24)};
        __builtin_nontemporal_store(w, (u32x2*)((uint8_t*)t.v + e0));
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (j < cnt) ((uint8_t*)t.v)[e0 + j] = (uint8_t)vc[j];
      }
    }
  }
}


// 2048-element block of a bf16 parameter with NF4 m and quad log-uint8 v
// (every large matrix of an LLM); a short last block is masked.  Same
// arithmetic as q8_block, organised for throughput:
//  * all 16 loads of the wavefront are issued before any math;
//  * SR off (the parity mode): exact IEEE divisions and midpoint comparisons,
//    identical to q8_block;
//  * SR on: random bits come from a per-lane xorshift32 stream seeded by a
//    keyed hash of (tensor, block, lane) -- 32 bits per element: bits 16-31 round
//    the bf16 parameter (v_cvt_sr_bf16_f32), bits 0-11 the NF4 code, bits 12-15
//    of the quad's first two elements its log-uint8 code; dequantisation is folded into the
//    momentum update (m' = code*ms*b1 + (1-b1)*g), the SNR gain into the quad's
//    reciprocal denominator, and a non-finite grad is detected from its quad's
//    sum of squares; the parameter update is one fma (p*decay - update) before
//    rounding; NF4 codes come from the signed fractional-index table:
//    code = (G(x) + r12) >> 12, two codes per 32-bit integer add, gathered
//    into bytes with v_perm_b32.
// The loads of one fast-path block: p and g (8 elements per lane per k), the NF4
// and log-uint8 code words and the block's two scales.
template <int PD> struct FastRaw {
  static constexpr int PW = PD == APEXW_F32 ? 2 : 1;   // 16-byte words of p / g per lane per k
  u32x4 pw[4][PW], gw[4][PW];
  uint32_t mw[4], vw[4];
  int cnt[4];
  float ms_old, vs_old;
};

// Block-uniform byte pointers of one 2048-element block (scalar registers: the
// tensor descriptor is read with scalar loads).  Element e = start + o of the
// block is addressed as base + 32-bit lane offset, so each access is one
// SGPR-base + VGPR-offset (+ immediate) instruction with no 64-bit VALU address
// arithmetic.
// The lane's offset passes through an empty asm statement in each block so the
// compiler does not hoist its 64-bit extension out of the unit loop (the
// SGPR-base form needs the 32-bit offset in the block that uses it).
template <int PD> struct FastBase {
  char* p;
  const char* g;
  uint8_t* m;
  uint8_t* v;
  uint32_t lane8;   // 8 * lane: the lane's first element in each 512-element group
  __device__ __forceinline__ FastBase(const apexw_tensor& t, int64_t start)
      : p((char*)t.p + start * Elem<PD>::bytes), g((const char*)t.g + start * Elem<PD>::bytes),
        m((uint8_t*)t.m + (start >> 1)), v((uint8_t*)t.v + (start >> 2)), lane8((uint32_t)lane_id() * 8u) {
    asm volatile("" : "+v"(lane8));
  }
};

template <int PD, bool FULL>
APEXW_DEV void q8_fast_load(const apexw_tensor& t, uint32_t blk, FastRaw<PD>& r) {
  constexpr int PW = FastRaw<PD>::PW;
  const int lane = lane_id();
  const int64_t start = (int64_t)blk * 2048;
  const FastBase<PD> fb(t, start);
  r.ms_old = t.m_scale[blk];
  r.vs_old = t.v_scale[blk];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t e = start + k * 512 + lane * 8;
    const uint32_t o = (uint32_t)(k * 512) + fb.lane8;   // element offset within the block
    const auto pp = APEXW_GLOBAL(const u32x4, fb.p + o * Elem<PD>::bytes);
    const auto gp = APEXW_GLOBAL(const u32x4, fb.g + o * Elem<PD>::bytes);
    if constexpr (FULL) {
      r.cnt[k] = 8;
#pragma unroll
      for (int h = 0; h < PW; ++h) {
        r.pw[k][h] = __builtin_nontemporal_load(pp + h);
        r.gw[k][h] = __builtin_nontemporal_load(gp + h);
      }
      r.mw[k] = __builtin_nontemporal_load(APEXW_GLOBAL(const uint32_t, fb.m + (o >> 1)));
      r.vw[k] = __builtin_nontemporal_load(APEXW_GLOBAL(const uint16_t, fb.v + (o >> 2)));
    } else {
      // numel % 4 == 0 for quad-v tensors, so a lane holds 0, 4 or 8 elements
      r.cnt[k] = e >= t.n ? 0 : (t.n - e >= 8 ? 8 : 4);
      const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int h = 0; h < PW; ++h) { r.pw[k][h] = z; r.gw[k][h] = z; }
      r.mw[k] = 0x77777777u; r.vw[k] = 0u;
      if (r.cnt[k] == 8) {
#pragma unroll
        for (int h = 0; h < PW; ++h) { r.pw[k][h] = pp[h]; r.gw[k][h] = gp[h]; }
        r.mw[k] = *APEXW_GLOBAL(const uint32_t, fb.m + (o >> 1));
        r.vw[k] = *APEXW_GLOBAL(const uint16_t, fb.v + (o >> 2));
      } else if (r.cnt[k] == 4) {
        if constexpr (PD == APEXW_F32) {
          r.pw[k][0] = pp[0];
          r.gw[k][0] = gp[0];
        } else {
          const u32x2 a = *APEXW_GLOBAL(const u32x2, fb.p + o * 2u);
          const u32x2 b = *APEXW_GLOBAL(const u32x2, fb.g + o * 2u);
          r.pw[k][0].x = a.x; r.pw[k][0].y = a.y; r.gw[k][0].x = b.x; r.gw[k][0].y = b.y;
        }
        r.mw[k] = 0x77770000u | *APEXW_GLOBAL(const uint16_t, fb.m + (o >> 1));
        r.vw[k] = *APEXW_GLOBAL(const uint8_t, fb.v + (o >> 2));
      }
    }
  }
}

// The arithmetic and stores of one fast-path block, from its loads.
// B1HI: the usual orientation of the two lerps, fixed at compile time (beta1 > 1/2:
// m' = lerp(m, g, 1-b1) takes the a + w (b - a) form and the lookahead lerp(g, m', b1)
// the b + (w - 1)(b - a) form); otherwise both come from the launch's flags.
template <int PD, bool SR, bool FULL, bool GENERIC, bool B1HI, bool GC>
APEXW_DEV void q8_fast_compute(const apexw_tensor& t, uint32_t tix, uint32_t blk, const Q8Ctx& c,
                               const FastRaw<PD>& r) {
  const apexw_hparams& hp = *c.hp;
  const uint32_t hf = hp.flags, tf = t.flags;
  const int lane = lane_id();
  const int64_t start = (int64_t)blk * 2048;
  const FastBase<PD> fb(t, start);
  const float ms_old = r.ms_old;
  const float vs_old = r.vs_old;
  const float decay = (tf & APEXW_FLAG_WD) ? hp.wd_factor : 1.0f;
  const bool lerp_hi = B1HI ? false : (bool)(hf & APEXW_HP_LERP_HI);
  const bool look_hi = B1HI ? true : (bool)(hf & APEXW_HP_LOOK_HI);
  const auto& pw = r.pw;
  const auto& gw = r.gw;
  const auto& mw = r.mw;
  const auto& vw = r.vw;
  const auto& cnt = r.cnt;
  uint32_t rs = 0;
  if constexpr (SR) {
    const uint32_t key = rng_key(hp.seed, tix, hp.step, 1u, (uint32_t)(start >> 32));
    rs = mix32(key + (blk << 6) + (uint32_t)lane) | 1u;
  }
  const bool prep = hf & (APEXW_HP_SANITIZE | APEXW_HP_CLIP | APEXW_HP_UNSCALE);
  BlockMeans bm{0, 0.0f, 0.0f, false, false};
  if constexpr (GC) bm = q8_block_means(c, t, start);

  // SR noise: one xorshift32 word per element pair in this pass (its two halves
  // round the pair's bf16 parameters) and one per pair in the requantization pass
  // (two 12-bit NF4 noises and 8 bits of v noise), drawn from the same stream there
  // rather than held in registers across the passes
  float mnew[4][8], vq[4][2];
  float amax = 0.0f, vmax = 0.0f;
  // SR path constants: (1 - b2) / 4 (exact), b2 * vs_old, and the step size times
  // each SNR gain
  const float omb2_q = hp.one_minus_beta2 * 0.25f, vsb2 = vs_old * hp.beta2;
  const float sg_hi = hp.step_size * c.gain_hi, sg_lo = hp.step_size * c.gain_lo;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float p[8], g[8], m[8];
    const uint32_t pv[4] = {pw[k][0].x, pw[k][0].y, pw[k][0].z, pw[k][0].w};
    float look[8];
    if constexpr (PD == APEXW_F32) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        p[4 * h] = __uint_as_float(pw[k][h].x); p[4 * h + 1] = __uint_as_float(pw[k][h].y);
        p[4 * h + 2] = __uint_as_float(pw[k][h].z); p[4 * h + 3] = __uint_as_float(pw[k][h].w);
        g[4 * h] = __uint_as_float(gw[k][h].x); g[4 * h + 1] = __uint_as_float(gw[k][h].y);
        g[4 * h + 2] = __uint_as_float(gw[k][h].z); g[4 * h + 3] = __uint_as_float(gw[k][h].w);
      }
    } else {
      const uint32_t gv[4] = {gw[k][0].x, gw[k][0].y, gw[k][0].z, gw[k][0].w};
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        p[2 * b] = __uint_as_float(pv[b] << 16);
        p[2 * b + 1] = __uint_as_float(pv[b] & 0xFFFF0000u);
        g[2 * b] = __uint_as_float(gv[b] << 16);
        g[2 * b + 1] = __uint_as_float(gv[b] & 0xFFFF0000u);
      }
    }
    if (prep) {
      if constexpr (GC) {
        const int64_t e = start + k * 512 + lane * 8;
        float mean[8];
        if (bm.by8) {
          const float mg = e < bm.split ? bm.m0 : bm.m1;
#pragma unroll
          for (int j = 0; j < 8; ++j) mean[j] = mg;
        } else if (bm.one) {
#pragma unroll
          for (int j = 0; j < 8; ++j) mean[j] = e + j < bm.split ? bm.m0 : bm.m1;
        } else {
          q8_means8(c, t, e, mean);
        }
        // the common case, centralization alone on finite grads (sanitizing changes
        // nothing): g - mean in the grad dtype; a non-finite difference (a non-finite
        // grad, or an overflow) sends the group through the general preparation
        float d[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) d[j] = rnd<PD>(g[j] - mean[j]);
        if (!(hf & (APEXW_HP_CLIP | APEXW_HP_UNSCALE)) && !q8_any_nonfinite8(d)) {
#pragma unroll
          for (int j = 0; j < 8; ++j) g[j] = d[j];
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) g[j] = q8_grad<PD>(g[j], tf, c, mean[j]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) g[j] = q8_grad<PD>(g[j], tf, c);
      }
    }
    float upd[8];
    if constexpr (SR) {
      // quad sums of squares first: a non-finite grad makes its quad's sum
      // non-finite, which sends the group through nan_to_num (rare path)
      float s2[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int b = 4 * q;
        float t = g[b] * g[b];
        t = fmaf(g[b + 1], g[b + 1], t);
        t = fmaf(g[b + 2], g[b + 2], t);
        s2[q] = fmaf(g[b + 3], g[b + 3], t);
      }
      if (!prep && !(__builtin_isfinite(s2[0]) && __builtin_isfinite(s2[1]))) {
#pragma unroll
        for (int j = 0; j < 8; ++j) g[j] = q8_grad<PD>(g[j], tf, c);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int b = 4 * q;
          float t = g[b] * g[b];
          t = fmaf(g[b + 1], g[b + 1], t);
          t = fmaf(g[b + 2], g[b + 2], t);
          s2[q] = fmaf(g[b + 3], g[b + 3], t);
        }
      }
      // m' = lerp(dequant(m), g, 1-b1) and the lookahead lerp(g, m', b1), rounded as torch's
      // lerp: the SNR gain switches on the sign of m' g, so m' must be the reference's value
      // to the last bit (an algebraically equal form can round a near-zero m' to the other sign)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float2 pr = c.pair[(mw[k] >> (8 * b)) & 0xFFu];
        m[2 * b] = lerp_to(pr.x * ms_old, g[2 * b], hp.lerp_coef, lerp_hi);
        m[2 * b + 1] = lerp_to(pr.y * ms_old, g[2 * b + 1], hp.lerp_coef, lerp_hi);
        look[2 * b] = lerp_to(g[2 * b], m[2 * b], hp.look_coef, look_hi);
        look[2 * b + 1] = lerp_to(g[2 * b + 1], m[2 * b + 1], hp.look_coef, look_hi);
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int b = 4 * q;
        // v' = b2 v + (1 - b2) mean4(g^2) with the block's b2 * vs_old and (1 - b2) / 4
        // folded into constants (within an fp32 ulp of the two-product form; SR only)
        float vv = fmaf(omb2_q, s2[q], c.vlut[(vw[k] >> (8 * q)) & 0xFFu] * vsb2);
        if (!(fabsf(vv) <= 3.402823466e38f)) vv = 0.0f;
        vq[k][q] = vv;
        if (FULL || 4 * q < cnt[k]) vmax = fmaxf(vmax, vv);
        const float r = __builtin_amdgcn_rcpf(fmaxf(__builtin_amdgcn_sqrtf(vv) + hp.eps_scaled, hp.eps));
        float r_hi = r * sg_hi, r_lo = r * sg_lo;
        // keep the two products per quad: otherwise the compiler sinks them below the
        // per-element select, one multiply per element instead of two per quad
        asm volatile("" : "+v"(r_hi), "+v"(r_lo));
#pragma unroll
        for (int i = 0; i < 4; ++i) upd[b + i] = look[b + i] * ((m[b + i] * g[b + i] >= 0.0f) ? r_hi : r_lo);
      }
    } else {
      // quad sums of squares (torch's mean over 4: three plain adds) first: a non-finite
      // grad makes its quad's sum non-finite, which sends the group through nan_to_num
      // (rare path; a finite grad whose square overflows goes through it unchanged)
      float s2[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int b = 4 * q;
        float t = g[b] * g[b];
        t = t + g[b + 1] * g[b + 1];
        t = t + g[b + 2] * g[b + 2];
        s2[q] = t + g[b + 3] * g[b + 3];
      }
      if (!prep && !(__builtin_isfinite(s2[0]) && __builtin_isfinite(s2[1]))) {
#pragma unroll
        for (int j = 0; j < 8; ++j) g[j] = q8_grad<PD>(g[j], tf, c);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int b = 4 * q;
          float t = g[b] * g[b];
          t = t + g[b + 1] * g[b + 1];
          t = t + g[b + 2] * g[b + 2];
          s2[q] = t + g[b + 3] * g[b + 3];
        }
      }
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float2 pr = c.pair[(mw[k] >> (8 * b)) & 0xFFu];
        m[2 * b] = pr.x * ms_old;
        m[2 * b + 1] = pr.y * ms_old;
      }
      float num[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        m[j] = lerp_to(m[j], g[j], hp.lerp_coef, lerp_hi);
        const float lk = lerp_to(g[j], m[j], hp.look_coef, look_hi);
        num[j] = lk * ((m[j] * g[j] >= 0.0f) ? c.gain_hi : c.gain_lo);
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int b = 4 * q;
        const float vold = c.vlut[(vw[k] >> (8 * q)) & 0xFFu] * vs_old;
        float vv = fmaf(hp.one_minus_beta2, s2[q] * 0.25f, vold * hp.beta2);
        if (!(fabsf(vv) <= 3.402823466e38f)) vv = 0.0f;
        vq[k][q] = vv;
        if (FULL || 4 * q < cnt[k]) vmax = fmaxf(vmax, vv);
        const float den = fmaxf(sqrtf(vv) + hp.eps_scaled, hp.eps);
        const float rden = rcp_refined(den);
#pragma unroll
        for (int i = 0; i < 4; ++i) upd[b + i] = div_shared(num[b + i], den, rden) * hp.step_size;
      }
    }
    const uint32_t o = (uint32_t)(k * 512) + fb.lane8;   // element offset within the block
    if constexpr (PD == APEXW_F32) {
      // fp32 parameters: p * decay - update in fp32 (both rounding orders agree), no SR
      float x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = p[j] * decay - upd[j];
      const u32x4 lo = {__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3])};
      const u32x4 hi = {__float_as_uint(x[4]), __float_as_uint(x[5]), __float_as_uint(x[6]), __float_as_uint(x[7])};
      const auto dst = APEXW_GLOBAL(u32x4, fb.p + o * 4u);
      if constexpr (FULL) {
        __builtin_nontemporal_store(lo, dst);
        __builtin_nontemporal_store(hi, dst + 1);
      } else if (cnt[k] == 8) {
        dst[0] = lo;
        dst[1] = hi;
      } else if (cnt[k] == 4) {
        dst[0] = lo;
      }
    } else {
    uint32_t pout[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if constexpr (SR) {
        // v_cvt_sr_bf16_f32 adds bits 16-31 of the random word to the fp32 pattern
        // and truncates (add-noise-then-truncate SR), writing one half of the pair:
        // the pair's word rounds its first element, the word's low half its second
        rs ^= rs << 13;
        rs ^= rs >> 17;
        rs ^= rs << 5;
        float y[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int j = 2 * b + i;
          y[i] = GENERIC ? rnd<APEXW_BF16>(p[j] * decay) - upd[j] : fmaf(p[j], decay, -upd[j]);
        }
        bf16x2 pr = __builtin_bit_cast(bf16x2, pv[b]);
        pr = __builtin_amdgcn_cvt_sr_bf16_f32(pr, y[0], rs, false);
        pr = __builtin_amdgcn_cvt_sr_bf16_f32(pr, y[1], rs << 16, true);
        pout[b] = __builtin_bit_cast(uint32_t, pr);
      } else {
        // the final rounding to bf16 is the pack itself (v_cvt_pk_bf16_f32, nearest-even)
        float x[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int j = 2 * b + i;
          if constexpr (GENERIC) {
            x[i] = rnd<APEXW_BF16>(p[j] * decay) - rnd<APEXW_BF16>(upd[j]);
          } else {
            x[i] = p[j] * decay - upd[j];
          }
        }
        pout[b] = pack_bf16x2(x[0], x[1]);
      }
    }
    u32x4 po = {pout[0], pout[1], pout[2], pout[3]};
    if constexpr (FULL) {
      __builtin_nontemporal_store(po, APEXW_GLOBAL(u32x4, fb.p + o * 2u));
    } else if (cnt[k] == 8) {
      *APEXW_GLOBAL(u32x4, fb.p + o * 2u) = po;
    } else if (cnt[k] == 4) {
      u32x2 p2 = {po.x, po.y};
      *APEXW_GLOBAL(u32x2, fb.p + o * 2u) = p2;
    }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      mnew[k][j] = m[j];
      if (FULL || j < cnt[k]) amax = fmaxf(amax, fabsf(m[j]));
    }
  }
  amax = wave_max(amax);
  vmax = wave_max(vmax);
  const float ms = fmaxf(fmaxf(amax, 1e-12f), ms_old * 0.9f);
  const float vs = fmaxf(fmaxf(vmax, 1e-12f), vs_old * 0.95f);
  if (lane == 0) {
    t.m_scale[blk] = ms;
    t.v_scale[blk] = vs;
  }
  const float rvs = __builtin_amdgcn_rcpf(vs);
  // SR: x = m / ms through the hardware reciprocal (within 1 ulp) shrunk by 2^-20, so
  // |x| <= (1 + 2^-23)(1 - 2^-20) < 1 - 2^-21 and y = x + 3 rounds inside [2, 4): the
  // code's bucket needs no clamp (the 2^-20 relative shrink is far below the code noise)
  const float rms_sr = __builtin_amdgcn_rcpf(ms) * 0x1.ffffep-1f;
  const float rms_rn = rcp_refined(ms), rvs_rn = rcp_refined(vs);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t o = (uint32_t)(k * 512) + fb.lane8;   // element offset within the block
    uint32_t w = 0;
    uint32_t hw[4];   // pair b: bits 0-11 / 16-27 NF4 noise, bits 12-15 / 28-31 v noise
    if constexpr (SR) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        rs ^= rs << 13;
        rs ^= rs >> 17;
        rs ^= rs << 5;
        hw[b] = rs;
      }
      uint32_t sum[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        uint32_t gc[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          // y = x + 3 for x = m / scale in (-1, 1): the top 7 mantissa bits of y in
          // [2, 4) are the bucket; the table is affine in y
          const float y = fmaf(mnew[k][2 * b + i], rms_sr, 3.0f);
          // byte 2 of y: its exponent bit (bit 23) is 0 in [2, 4), so this is the
          // 7-bit bucket, read with one byte-select shift (the table has 256 entries,
          // the upper half a copy, so any byte stays inside it)
          const float4 fr = c.frac16[(__float_as_uint(y) >> 16) & 255u];
          gc[i] = (uint32_t)fabsf(fminf(fmaf(fr.y, y, fr.x), fmaf(fr.w, y, fr.z)));
        }
        // two 16-bit lanes of G + r12 (r12 = bits 0-11 of the element's word):
        // the stochastic code lands in bits 12-15 and 28-31
        sum[b] = (gc[0] | (gc[1] << 16)) + (hw[b] & 0x0FFF0FFFu);
      }
      // gather bytes 1 and 3 (code << 4 | noise) of the four pair sums, then
      // byte b = code[2b] << 4 | code[2b+1]
      const uint32_t lo01 = __builtin_amdgcn_perm(sum[1], sum[0], 0x07030501u);  // s0.b1 s1.b1 s0.b3 s1.b3
      const uint32_t lo23 = __builtin_amdgcn_perm(sum[3], sum[2], 0x07030501u);
      const uint32_t even = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);      // code[2b] in high nibbles
      const uint32_t odd = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);       // code[2b+1] in high nibbles
      w = (even & 0xF0F0F0F0u) | ((odd >> 4) & 0x0F0F0F0Fu);
    } else {
      uint32_t code[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        code[j] = nf4_rne_tab(fminf(fmaxf(div_shared(mnew[k][j], ms, rms_rn), -1.0f), 1.0f), c.midtab);
#pragma unroll
      for (int b = 0; b < 4; ++b) w |= ((code[2 * b] << 4) | code[2 * b + 1]) << (8 * b);
    }
    uint32_t vc[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float vv = vq[k][q];
      if (!(vv > 0.0f)) {
        vc[q] = 0u;
      } else if constexpr (SR) {
        const float r = fmaxf(vv * rvs, 0x1p-24f);
        // bits 12-15 of the quad's first two words -> 8 bits -> u = (r + 1/2) / 2^8, then floor
        const uint32_t a = hw[2 * q];
        const uint32_t r8 = ((a >> 12) & 0xFu) | ((a >> 24) & 0xF0u);
        const float u = __uint_as_float(0x3F804000u | (r8 << 15)) - 1.0f;
        const float qf = fmaf(__builtin_amdgcn_logf(r), 0x1.52aaaap+3f, 255.0f) + u;
        vc[q] = (uint32_t)__builtin_amdgcn_fmed3f(qf, 1.0f, 255.0f);
      } else {
        vc[q] = logu8_code_shared(vv, vs, rvs_rn);
      }
    }
    if constexpr (FULL) {
      __builtin_nontemporal_store(w, APEXW_GLOBAL(uint32_t, fb.m + (o >> 1)));
      __builtin_nontemporal_store((uint16_t)(vc[0] | (vc[1] << 8)), APEXW_GLOBAL(uint16_t, fb.v + (o >> 2)));
    } else if (cnt[k] == 8) {
      *APEXW_GLOBAL(uint32_t, fb.m + (o >> 1)) = w;
      *APEXW_GLOBAL(uint16_t, fb.v + (o >> 2)) = (uint16_t)(vc[0] | (vc[1] << 8));
    } else if (cnt[k] == 4) {
      *APEXW_GLOBAL(uint16_t, fb.m + (o >> 1)) = (uint16_t)(w & 0xFFFFu);
      *APEXW_GLOBAL(uint8_t, fb.v + (o >> 2)) = (uint8_t)vc[0];
    }
  }
}

template <int PD, bool SR, bool FULL, bool GENERIC, bool B1HI, bool GC>
APEXW_DEV void q8_block_fast(const apexw_tensor& t, uint32_t tix, uint32_t blk, const Q8Ctx& c) {
  FastRaw<PD> r;
  q8_fast_load<PD, FULL>(t, blk, r);
  q8_fast_compute<PD, SR, FULL, GENERIC, B1HI, GC>(t, tix, blk, c, r);
}

// Dense m and v (bf16 or fp32): the fallback branch of _step_ultra
// (optimizer.py:4688-4735) for 8-bit tensors under 64 elements and the small
// tensors of precision "ultra" (fp32 m/v).  One 2048-element unit per wave,
// one element per lane at a time (these tensors are small).
// SINGLE: the per-parameter in-backward update of such a tensor
// (apexw/optimizer.py:2458-2471): p.mul_(wd) in the parameter dtype, fp32
// moments, p.addcdiv_ rounded once, m and v rounded once on store.
template <int PD, int MD, int VD, bool SINGLE>
APEXW_DEV void q8_dense(const apexw_tensor& t, uint32_t unit, const Q8Ctx& c) {
  constexpr int GD = PD;
  const apexw_hparams& hp = *c.hp;
  const int64_t start = (int64_t)unit * 2048;
  const int64_t end = (t.n - start) < 2048 ? t.n : start + 2048;
  for (int64_t i = start + lane_id(); i < end; i += 64) {
    float p = load1<PD>(t.p, i);
    if constexpr (SINGLE) {
      const float g = load1<GD>(t.g, i);
      if (t.flags & APEXW_FLAG_WD) p = rnd<PD>(p * hp.wd_factor);
      const float mf = fmaf(hp.one_minus_beta1, g, load1<MD>(t.m, i) * hp.beta1);
      const float vf = fmaf(hp.one_minus_beta2 * g, g, load1<VD>(t.v, i) * hp.beta2);
      const float den = sqrtf(vf) + hp.eps_scaled;
      store1<MD>(t.m, i, rnd<MD>(mf));
      store1<VD>(t.v, i, rnd<VD>(vf));
      store1<PD>(t.p, i, rnd<PD>(p + (-hp.step_size * mf) / den));
      continue;
    }
    const float g = q8_grad<GD>(load1<GD>(t.g, i), t.flags, c, q8_mean1(c, t, i));
    if (t.flags & APEXW_FLAG_WD) p = rnd<PD>(p * hp.wd_factor);
    const float mf = lerp_to(load1<MD>(t.m, i), g, hp.lerp_coef, hp.flags & APEXW_HP_LERP_HI);
    store1<MD>(t.m, i, rnd<MD>(mf));
    const float vf = fmaf(hp.one_minus_beta2 * g, g, load1<VD>(t.v, i) * hp.beta2);
    store1<VD>(t.v, i, rnd<VD>(vf));
    const float den = sqrtf(vf) + hp.eps_scaled;
    // Nesterov: torch.lerp(g, m, beta1) on the fp32 m (optimizer.py:4719-4724)
    float num = (hp.flags & APEXW_HP_NESTEROV) ? lerp_to(g, mf, hp.look_coef, hp.flags & APEXW_HP_LOOK_HI) : mf;
    // cautious: num * (mask / mean(mask)), mask = num g >= 0 (optimizer.py:4726-4729)
    if (hp.flags & APEXW_HP_CAUTIOUS) num = num * ((num * g >= 0.0f) ? c.gain_hi : 0.0f);
    const float upd = (num / den) * hp.step_size;
    if constexpr (PD == APEXW_F32) p = p - upd;
    else p = rnd<PD>(p - rnd<PD>(upd));
    store1<PD>(t.p, i, p);
  }
}

// Precision "ultra" (optimizer.py:4640-4686): one INT8 block of m per wave
// (t.block = 2048 or 256 elements, scales EMA-max smoothed as for 8-bit) and a
// dense v in VD.  m = lerp(dequant(m), g, 1 - beta1); v = beta2 v + (1 - beta2) g^2
// in fp32, stored rounded to VD; the denominator sqrt(v) + eps_scaled comes from
// the unrounded v, with no eps floor and no lookahead gain; p is decayed (rounded
// to its dtype), then p - update rounded to p's dtype.
template <int PD, int VD>
APEXW_DEV void ultra_block(const apexw_tensor& t, uint32_t tix, uint32_t blk, const Q8Ctx& c) {
  constexpr int GD = PD;
  const apexw_hparams& hp = *c.hp;
  const bool sr = hp.flags & APEXW_HP_SR;
  const bool vec = !(t.flags & APEXW_FLAG_SCALAR);
  const int64_t bs = t.block;
  const int64_t start = (int64_t)blk * bs;
  const int64_t cnt_blk = (t.n - start) < bs ? (t.n - start) : bs;
  const int lane = lane_id();
  const float ms_old = t.m_scale[blk];
  const uint32_t key = rng_key(hp.seed, tix, hp.step, 1u, (uint32_t)(start >> 32));
  float mnew[4][8];
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t rel = (int64_t)(k * 64 + lane) * 8;
    const int cnt = rel >= cnt_blk ? 0 : (int)((cnt_blk - rel) < 8 ? (cnt_blk - rel) : 8);
#pragma unroll
    for (int j = 0; j < 8; ++j) mnew[k][j] = 0.0f;
    if (cnt == 0) continue;
    const int64_t e0 = start + rel;
    const bool full = vec && cnt == 8;
    float p[8], g[8], m[8], v[8];
    if (full) {
      load8<PD>(t.p, e0, p);
      load8<GD>(t.g, e0, g);
      load8<VD>(t.v, e0, v);
      const u32x2 w = __builtin_nontemporal_load((const u32x2*)((const int8_t*)t.m + e0));
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t word = j < 4 ? w.x : w.y;
        m[j] = (float)(int8_t)((word >> (8 * (j & 3))) & 0xFFu) * ms_old;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool ok = j < cnt;
        p[j] = ok ? load1<PD>(t.p, e0 + j) : 0.0f;
        g[j] = ok ? load1<GD>(t.g, e0 + j) : 0.0f;
        v[j] = ok ? load1<VD>(t.v, e0 + j) : 0.0f;
        m[j] = ok ? (float)((const int8_t*)t.m)[e0 + j] * ms_old : 0.0f;
      }
    }
    float mean[8];
    q8_means8(c, t, e0, mean);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      g[j] = q8_grad<GD>(g[j], t.flags, c, mean[j]);
      if (t.flags & APEXW_FLAG_WD) p[j] = rnd<PD>(p[j] * hp.wd_factor);
      m[j] = lerp_to(m[j], g[j], hp.lerp_coef, hp.flags & APEXW_HP_LERP_HI);
      const float vf = fmaf(hp.one_minus_beta2 * g[j], g[j], v[j] * hp.beta2);
      v[j] = rnd<VD>(vf);
      // Nesterov: torch.lerp(g, m, beta1) on the fp32 m (optimizer.py:4667-4670)
      float num = (hp.flags & APEXW_HP_NESTEROV)
                      ? lerp_to(g[j], m[j], hp.look_coef, hp.flags & APEXW_HP_LOOK_HI) : m[j];
      // cautious: num * (mask / mean(mask)), mask = num g >= 0 (optimizer.py:4672-4675)
      if (hp.flags & APEXW_HP_CAUTIOUS) num = num * ((num * g[j] >= 0.0f) ? c.gain_hi : 0.0f);
      const float upd = (num / (sqrtf(vf) + hp.eps_scaled)) * hp.step_size;
      if constexpr (PD == APEXW_F32) p[j] = p[j] - upd;
      else p[j] = rnd<PD>(p[j] - rnd<PD>(upd));
    }
    if (full) {
      store8<PD>(t.p, e0, p);
      store8<VD>(t.v, e0, v);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j < cnt) {
          store1<PD>(t.p, e0 + j, p[j]);
          store1<VD>(t.v, e0 + j, v[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < cnt) {
        mnew[k][j] = m[j];
        amax = fmaxf(amax, fabsf(m[j]));
      }
    }
  }
  // the block scale and the INT8 codes, as the 8-bit step's (quantize_blockwise_int8)
  amax = wave_max(amax);
  const float ms = fmaxf(fmaxf(amax, 1e-12f) / 127.0f, ms_old * 0.9f);
  if (lane == 0) t.m_scale[blk] = ms;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t rel = (int64_t)(k * 64 + lane) * 8;
    const int cnt = rel >= cnt_blk ? 0 : (int)((cnt_blk - rel) < 8 ? (cnt_blk - rel) : 8);
    if (cnt == 0) continue;
    const int64_t e0 = start + rel;
    uint32_t mc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float y = mnew[k][j] / ms;
      if (sr) y = y + (unit_uniform(rng_at(key, (uint32_t)(e0 + j)) >> 16) - 0.5f);
      y = fminf(fmaxf(rintf(y), -127.0f), 127.0f);
      mc[j] = (uint32_t)(int32_t)y & 0xFFu;
    }
    if (vec && cnt == 8) {
      u32x2 w = {mc[0] | (mc[1] << 8) | (mc[2] << 16) | (mc[3] << 24),
                 mc[4] | (mc[5] << 8) | (mc[6] << 16) | (mc[7] << 24)};
      __builtin_nontemporal_store(w, (u32x2*)((int8_t*)t.m + e0));
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < cnt) ((uint8_t*)t.m)[e0 + j] = (uint8_t)mc[j];
    }
  }
}


// Raw 16-byte loads of 8 consecutive elements of dtype DT (two for fp32), and
// their values.
template <int DT> struct Raw8 {
  u32x4 w[DT == APEXW_F32 ? 2 : 1];
};
template <int DT> APEXW_DEV void raw_load8(const void* base, int64_t i, Raw8<DT>& r) {
  if constexpr (DT == APEXW_F32) {
    auto p = APEXW_GLOBAL(const u32x4, (const float*)base + i);
    r.w[0] = __builtin_nontemporal_load(p);
    r.w[1] = __builtin_nontemporal_load(p + 1);
  } else {
    r.w[0] = __builtin_nontemporal_load(APEXW_GLOBAL(const u32x4, (const uint16_t*)base + i));
  }
}
template <int DT> APEXW_DEV void unpack8(const Raw8<DT>& r, float (&x)[8]) {
#pragma unroll
  for (int q = 0; q < (DT == APEXW_F32 ? 2 : 1); ++q) {
    const uint32_t w[4] = {r.w[q].x, r.w[q].y, r.w[q].z, r.w[q].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (DT == APEXW_F32) {
        x[4 * q + k] = __uint_as_float(w[k]);
      } else if constexpr (DT == APEXW_BF16) {
        x[2 * k] = bf16_bits_to_f32(w[k] & 0xFFFFu);
        x[2 * k + 1] = __uint_as_float(w[k] & 0xFFFF0000u);
      } else {
        x[2 * k] = f16_bits_to_f32(w[k] & 0xFFFFu);
        x[2 * k + 1] = f16_bits_to_f32(w[k] >> 16);
      }
    }
  }
}

// A whole 2048-element "ultra" block (the arithmetic of ultra_block): the loads of
// KB of the wave's four 8-element groups per lane are issued before their
// arithmetic (all four for bf16 p and v, two at a time when p or v is fp32), so the
// block waits on memory once or twice instead of four times.
template <int PD, int VD>
APEXW_DEV void ultra_block_full(const apexw_tensor& t, uint32_t tix, uint32_t blk, const Q8Ctx& c) {
  constexpr int GD = PD;
  constexpr int KB = (PD == APEXW_F32 || VD == APEXW_F32) ? 2 : 4;
  const apexw_hparams& hp = *c.hp;
  const bool sr = hp.flags & APEXW_HP_SR;
  const bool wd = t.flags & APEXW_FLAG_WD;
  const int64_t start = (int64_t)blk * 2048;
  const int lane = lane_id();
  const float ms_old = t.m_scale[blk];
  const uint32_t key = rng_key(hp.seed, tix, hp.step, 1u, (uint32_t)(start >> 32));
  float mnew[4][8];
  float amax = 0.0f;
#pragma unroll
  for (int k0 = 0; k0 < 4; k0 += KB) {
    Raw8<PD> rp[KB];
    Raw8<GD> rg[KB];
    Raw8<VD> rv[KB];
    u32x2 rm[KB];
#pragma unroll
    for (int b = 0; b < KB; ++b) {
      const int64_t e0 = start + (int64_t)((k0 + b) * 64 + lane) * 8;
      raw_load8<PD>(t.p, e0, rp[b]);
      raw_load8<GD>(t.g, e0, rg[b]);
      raw_load8<VD>(t.v, e0, rv[b]);
      rm[b] = __builtin_nontemporal_load(APEXW_GLOBAL(const u32x2, (const int8_t*)t.m + e0));
    }
#pragma unroll
    for (int b = 0; b < KB; ++b) {
      const int k = k0 + b;
      const int64_t e0 = start + (int64_t)(k * 64 + lane) * 8;
      float p[8], g[8], v[8];
      unpack8<PD>(rp[b], p);
      unpack8<GD>(rg[b], g);
      unpack8<VD>(rv[b], v);
      float mean[8];
      q8_means8(c, t, e0, mean);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t word = j < 4 ? rm[b].x : rm[b].y;
        const float m = (float)(int8_t)((word >> (8 * (j & 3))) & 0xFFu) * ms_old;
        g[j] = q8_grad<GD>(g[j], t.flags, c, mean[j]);
        if (wd) p[j] = rnd<PD>(p[j] * hp.wd_factor);
        mnew[k][j] = lerp_to(m, g[j], hp.lerp_coef, hp.flags & APEXW_HP_LERP_HI);
        amax = fmaxf(amax, fabsf(mnew[k][j]));
        const float vf = fmaf(hp.one_minus_beta2 * g[j], g[j], v[j] * hp.beta2);
        v[j] = rnd<VD>(vf);
        float num = (hp.flags & APEXW_HP_NESTEROV)
                        ? lerp_to(g[j], mnew[k][j], hp.look_coef, hp.flags & APEXW_HP_LOOK_HI) : mnew[k][j];
        if (hp.flags & APEXW_HP_CAUTIOUS) num = num * ((num * g[j] >= 0.0f) ? c.gain_hi : 0.0f);
        const float upd = (num / (sqrtf(vf) + hp.eps_scaled)) * hp.step_size;
        if constexpr (PD == APEXW_F32) p[j] = p[j] - upd;
        else p[j] = rnd<PD>(p[j] - rnd<PD>(upd));
      }
      store8<PD>(t.p, e0, p);
      store8<VD>(t.v, e0, v);
    }
  }
  amax = wave_max(amax);
  const float ms = fmaxf(fmaxf(amax, 1e-12f) / 127.0f, ms_old * 0.9f);
  if (lane == 0) t.m_scale[blk] = ms;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t e0 = start + (int64_t)(k * 64 + lane) * 8;
    uint32_t mc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float y = mnew[k][j] / ms;
      if (sr) y = y + (unit_uniform(rng_at(key, (uint32_t)(e0 + j)) >> 16) - 0.5f);
      y = fminf(fmaxf(rintf(y), -127.0f), 127.0f);
      mc[j] = (uint32_t)(int32_t)y & 0xFFu;
    }
    u32x2 w = {mc[0] | (mc[1] << 8) | (mc[2] << 16) | (mc[3] << 24),
               mc[4] | (mc[5] << 8) | (mc[6] << 16) | (mc[7] << 24)};
    __builtin_nontemporal_store(w, (u32x2*)((int8_t*)t.m + e0));
  }
}

template <int PD, int VD>
APEXW_DEV void ultra_unit(const apexw_tensor& t, uint32_t tix, uint32_t blk, const Q8Ctx& c) {
  const bool whole = t.block == 2048 && (int64_t)(blk + 1) * 2048 <= t.n && !(t.flags & APEXW_FLAG_SCALAR);
  if (whole) ultra_block_full<PD, VD>(t, tix, blk, c);
  else ultra_block<PD, VD>(t, tix, blk, c);
}

// Dense m / v rows by dtype: m in the parameter's compact dtype (bf16; fp16 for fp16
// parameters) with v in it or fp32, or fp32 m and v.
template <bool SINGLE>
APEXW_DEV void dense_dispatch(const apexw_tensor& t, uint32_t unit, const Q8Ctx& c, uint32_t pd, uint32_t md,
                              uint32_t vd) {
  if (md == APEXW_F32) {
    // fp32 m implies fp32 v (checked on the host)
    if (pd == APEXW_F32) q8_dense<APEXW_F32, APEXW_F32, APEXW_F32, SINGLE>(t, unit, c);
    else if (pd == APEXW_BF16) q8_dense<APEXW_BF16, APEXW_F32, APEXW_F32, SINGLE>(t, unit, c);
    else q8_dense<APEXW_F16, APEXW_F32, APEXW_F32, SINGLE>(t, unit, c);
  } else if (pd == APEXW_F32) {
    if (vd == APEXW_F32) q8_dense<APEXW_F32, APEXW_BF16, APEXW_F32, SINGLE>(t, unit, c);
    else q8_dense<APEXW_F32, APEXW_BF16, APEXW_BF16, SINGLE>(t, unit, c);
  } else if (pd == APEXW_BF16) {
    if (vd == APEXW_F32) q8_dense<APEXW_BF16, APEXW_BF16, APEXW_F32, SINGLE>(t, unit, c);
    else q8_dense<APEXW_BF16, APEXW_BF16, APEXW_BF16, SINGLE>(t, unit, c);
  } else {
    if (vd == APEXW_F32) q8_dense<APEXW_F16, APEXW_F16, APEXW_F32, SINGLE>(t, unit, c);
    else q8_dense<APEXW_F16, APEXW_F16, APEXW_F16, SINGLE>(t, unit, c);
  }
}

// The "ultra" precision's step: its INT8-m blocks (APEXW_FLAG_ULTRA) and its small
// tensors' dense fp32 m / v (APEXW_FLAG_DENSE), in a kernel of their own so that the
// general 8-bit kernel's NF4 / log-uint8 code does not set its register count.
// Rows of any other kind are not this kernel's (the host never lists them).
__global__ __launch_bounds__(256) void ultra_step_kernel(const apexw_tensor* __restrict__ tensors,
                                                         const apexw_unit* __restrict__ units, int64_t n_units,
                                                         apexw_hparams hp_in) {
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
  Q8Ctx c;
  c.hp = &hp;
  c.vlut = nullptr;
  c.code = nullptr;
  c.pair = nullptr;
  c.frac16 = nullptr;
  c.midtab = nullptr;
  c.coef = (hp.flags & APEXW_HP_CLIP) ? *hp.clip_coef : 1.0f;
  c.gc_means = nullptr;
  c.gc_rl = 0;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const int64_t stride = (int64_t)gridDim.x * kWaves;
  for (int64_t u = (int64_t)blockIdx.x * kWaves + wave; u < n_units; u += stride) {
    const apexw_unit un = units[u];
    const apexw_tensor& t = tensors[un.tensor];
    q8_set_rows(c, t, un.tensor);
    q8_set_gains(c, t, un.tensor);
    const uint32_t f = t.flags;
    const uint32_t pd = (f >> APEXW_FLAG_PDT_SHIFT) & 3u;
    const uint32_t md = (f >> APEXW_FLAG_MDT_SHIFT) & 3u;
    const uint32_t vd = (f >> APEXW_FLAG_VDT_SHIFT) & 3u;
    if (f & APEXW_FLAG_DENSE) {
      dense_dispatch<false>(t, un.unit, c, pd, md, vd);
    } else if (f & APEXW_FLAG_ULTRA) {
      // v in the parameter's compact dtype (fp16 for fp16 parameters, else bf16) or fp32
      if (pd == APEXW_F32) {
        if (vd == APEXW_F32) ultra_unit<APEXW_F32, APEXW_F32>(t, un.tensor, un.unit, c);
        else ultra_unit<APEXW_F32, APEXW_BF16>(t, un.tensor, un.unit, c);
      } else if (pd == APEXW_BF16) {
        if (vd == APEXW_F32) ultra_unit<APEXW_BF16, APEXW_F32>(t, un.tensor, un.unit, c);
        else ultra_unit<APEXW_BF16, APEXW_BF16>(t, un.tensor, un.unit, c);
      } else {
        if (vd == APEXW_F32) ultra_unit<APEXW_F16, APEXW_F32>(t, un.tensor, un.unit, c);
        else ultra_unit<APEXW_F16, APEXW_F16>(t, un.tensor, un.unit, c);
      }
    }
  }
}


// Kernel for the units of fast-path tensors (see apexw_q8_fast_ok) with parameter
// dtype PD and stochastic rounding SR; each (dtype, SR) pair is its own kernel so
// one variant's register footprint does not lower another's occupancy (bf16: 142
// VGPRs with SR, occupancy 3; 93 without, occupancy 5).  GC: the launch holds
// centralized tensors (hparams.rows), an instantiation of its own so that the
// others keep their register counts.
template <int PD, bool SR, bool B1HI, bool GC>
__global__ __launch_bounds__(256) void q8_fast_kernel(const apexw_tensor* __restrict__ tensors,
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
  __shared__ float s_vlut[256];
  __shared__ float2 s_pair[256];
  __shared__ float4 s_frac16[256];   // 128 buckets, then a copy of them
  __shared__ float2 s_midtab[64];
  s_vlut[threadIdx.x] = kVLogLut[threadIdx.x];
  if (threadIdx.x < 64) s_midtab[threadIdx.x] = make_float2(kNf4MidTab[2 * threadIdx.x], kNf4MidTab[2 * threadIdx.x + 1]);
  s_pair[threadIdx.x] = make_float2(kNf4Pair[2 * threadIdx.x], kNf4Pair[2 * threadIdx.x + 1]);
  {
    const int f = threadIdx.x & 127;
    s_frac16[threadIdx.x] = make_float4(kNf4Code16[4 * f], kNf4Code16[4 * f + 1], kNf4Code16[4 * f + 2],
                                        kNf4Code16[4 * f + 3]);
  }
  __syncthreads();
  Q8Ctx c;
  c.hp = &hp;
  c.vlut = s_vlut;
  c.code = nullptr;
  c.pair = s_pair;
  c.frac16 = s_frac16;
  c.midtab = s_midtab;
  c.coef = (hp.flags & APEXW_HP_CLIP) ? *hp.clip_coef : 1.0f;
  c.gc_means = nullptr;
  c.gc_rl = 0;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  // a workgroup walks a contiguous chunk of kFastChunk units, its waves interleaved
  // (unit base + 4 i + wave): measured ~1% faster than workgroups striding by 4 units
  for (int64_t base = (int64_t)blockIdx.x * kFastChunk; base < n_units; base += (int64_t)gridDim.x * kFastChunk)
  for (int64_t u = base + wave, u_end = base + kFastChunk < n_units ? base + kFastChunk : n_units; u < u_end;
       u += kWaves) {
    const apexw_unit un = units[u];
    const apexw_tensor& t = tensors[un.tensor];
    // never taken for a valid plan: the unit ranges hold only this kernel's tensors
    if (!apexw_q8_fast_ok(t.flags, t.block) || ((t.flags >> APEXW_FLAG_PDT_SHIFT) & 3u) != (uint32_t)PD) continue;
    if constexpr (GC) q8_set_rows(c, t, un.tensor);
    q8_set_gains(c, t, un.tensor);
    const bool full = (int64_t)(un.unit + 1) * 2048 <= t.n;
    const bool gen = t.flags & APEXW_FLAG_GENERIC;
    if (full && !gen) q8_block_fast<PD, SR, true, false, B1HI, GC>(t, un.tensor, un.unit, c);
    else if (full) q8_block_fast<PD, SR, true, true, B1HI, GC>(t, un.tensor, un.unit, c);
    else if (!gen) q8_block_fast<PD, SR, false, false, B1HI, GC>(t, un.tensor, un.unit, c);
    else q8_block_fast<PD, SR, false, true, B1HI, GC>(t, un.tensor, un.unit, c);
  }
}

template <bool SINGLE>
__global__ __launch_bounds__(256) void q8_step_kernel(const apexw_tensor* __restrict__ tensors,
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
  __shared__ float s_vlut[256];
  __shared__ float s_code[16];
  __shared__ float2 s_midtab[64];
  s_vlut[threadIdx.x] = kVLogLut[threadIdx.x];
  if (threadIdx.x < 16) s_code[threadIdx.x] = kNf4Code[threadIdx.x];
  if (threadIdx.x < 64) s_midtab[threadIdx.x] = make_float2(kNf4MidTab[2 * threadIdx.x], kNf4MidTab[2 * threadIdx.x + 1]);
  __syncthreads();
  Q8Ctx c;
  c.hp = &hp;
  c.vlut = s_vlut;
  c.code = s_code;
  c.pair = nullptr;
  c.frac16 = nullptr;
  c.midtab = s_midtab;
  c.coef = (hp.flags & APEXW_HP_CLIP) ? *hp.clip_coef : 1.0f;
  c.gc_means = nullptr;
  c.gc_rl = 0;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const int64_t stride = (int64_t)gridDim.x * kWaves;
  for (int64_t u = (int64_t)blockIdx.x * kWaves + wave; u < n_units; u += stride) {
    const apexw_unit un = units[u];
    const apexw_tensor& t = tensors[un.tensor];
    q8_set_rows(c, t, un.tensor);
    q8_set_gains(c, t, un.tensor);
    const uint32_t f = t.flags;
    const uint32_t pd = (f >> APEXW_FLAG_PDT_SHIFT) & 3u;
    if (f & APEXW_FLAG_FACTORED) continue;  // stepped by apexw_factored_step
    const uint32_t vd = (f >> APEXW_FLAG_VDT_SHIFT) & 3u;
    if (f & APEXW_FLAG_DENSE) {
      dense_dispatch<SINGLE>(t, un.unit, c, pd, (f >> APEXW_FLAG_MDT_SHIFT) & 3u, vd);
      continue;
    }
    // ultra rows belong to ultra_step_kernel (apexw_ultra_step): never read their dense v as codes
    if (f & APEXW_FLAG_ULTRA) continue;
    const bool nf4 = f & APEXW_FLAG_NF4, quad = f & APEXW_FLAG_QUAD;
    if (pd == APEXW_F32) {
      if (nf4 && quad) q8_block<APEXW_F32, true, true, SINGLE>(t, un.tensor, un.unit, c);
      else if (nf4) q8_block<APEXW_F32, true, false, SINGLE>(t, un.tensor, un.unit, c);
      else q8_block<APEXW_F32, false, false, SINGLE>(t, un.tensor, un.unit, c);
    } else if (pd == APEXW_BF16) {
      if (nf4 && quad) q8_block<APEXW_BF16, true, true, SINGLE>(t, un.tensor, un.unit, c);
      else if (nf4) q8_block<APEXW_BF16, true, false, SINGLE>(t, un.tensor, un.unit, c);
      else q8_block<APEXW_BF16, false, false, SINGLE>(t, un.tensor, un.unit, c);
    } else {
      if (nf4 && quad) q8_block<APEXW_F16, true, true, SINGLE>(t, un.tensor, un.unit, c);
      else if (nf4) q8_block<APEXW_F16, true, false, SINGLE>(t, un.tensor, un.unit, c);
      else q8_block<APEXW_F16, false, false, SINGLE>(t, un.tensor, un.unit, c);
    }
  }
}

// cautious=True: per descriptor, the number of elements whose updated first
// moment m' = lerp(m, g', 1 - beta1) has m' g' >= 0 (the reference's mask, whose
// mean scales the numerator: apexw/optimizer.py:4585-4588, :4672-4675, :4726-4729),
// g' the grad as the step prepares it.  One unit per wave (a quantization block, or
// 2048 elements of a dense row), one element per lane at a time; one atomic add of
// the wave's count per unit.
__global__ __launch_bounds__(256) void q8_cautious_count_kernel(const apexw_tensor* __restrict__ tensors,
                                                                const apexw_unit* __restrict__ units,
                                                                int64_t n_units, apexw_hparams hp_in) {
  apexw_hparams hp = hp_in;
  if (hp.flags & APEXW_HP_AMP) {
    const apexw_amp_dyn d = *hp.amp;
    if (d.skip) return;
    hp.grad_inv_scale = d.grad_inv_scale;
  }
  __shared__ float s_code[16];
  if (threadIdx.x < 16) s_code[threadIdx.x] = kNf4Code[threadIdx.x];
  __syncthreads();
  Q8Ctx c;
  c.hp = &hp;
  c.vlut = nullptr;
  c.code = s_code;
  c.pair = nullptr;
  c.frac16 = nullptr;
  c.midtab = nullptr;
  c.coef = (hp.flags & APEXW_HP_CLIP) ? *hp.clip_coef : 1.0f;
  c.gc_means = nullptr;
  c.gc_rl = 0;
  c.gain_hi = c.gain_lo = 0.0f;
  const bool lerp_hi = hp.flags & APEXW_HP_LERP_HI;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const int lane = lane_id();
  const int64_t stride = (int64_t)gridDim.x * kWaves;
  for (int64_t u = (int64_t)blockIdx.x * kWaves + wave; u < n_units; u += stride) {
    const apexw_unit un = units[u];
    const apexw_tensor& t = tensors[un.tensor];
    const uint32_t f = t.flags;
    if (f & APEXW_FLAG_FACTORED) continue;
    q8_set_rows(c, t, un.tensor);
    const uint32_t pd = (f >> APEXW_FLAG_PDT_SHIFT) & 3u, md = (f >> APEXW_FLAG_MDT_SHIFT) & 3u;
    const bool dense = f & APEXW_FLAG_DENSE, nf4 = f & APEXW_FLAG_NF4;
    const int64_t bs = dense ? 2048 : (int64_t)t.block;
    const int64_t start = (int64_t)un.unit * bs, end = (t.n - start) < bs ? t.n : start + bs;
    const float ms = dense ? 0.0f : t.m_scale[un.unit];
    uint32_t cnt = 0;
    for (int64_t i = start + lane; i < end; i += 64) {
      const float mean = q8_mean1(c, t, i);
      float g;
      if (pd == APEXW_F32) g = q8_grad<APEXW_F32>(load1<APEXW_F32>(t.g, i), f, c, mean);
      else if (pd == APEXW_BF16) g = q8_grad<APEXW_BF16>(load1<APEXW_BF16>(t.g, i), f, c, mean);
      else g = q8_grad<APEXW_F16>(load1<APEXW_F16>(t.g, i), f, c, mean);
      float m;
      if (dense) {
        m = md == APEXW_F32 ? load1<APEXW_F32>(t.m, i)
                            : (md == APEXW_BF16 ? load1<APEXW_BF16>(t.m, i) : load1<APEXW_F16>(t.m, i));
      } else if (nf4) {
        const uint32_t byte = ((const uint8_t*)t.m)[i >> 1];
        m = c.code[(i & 1) ? (byte & 15u) : (byte >> 4)] * ms;
      } else {
        m = (float)((const int8_t*)t.m)[i] * ms;
      }
      const float mn = lerp_to(m, g, hp.lerp_coef, lerp_hi);
      cnt += (mn * g >= 0.0f) ? 1u : 0u;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
    if (lane == 0 && cnt) atomicAdd(&hp.counts[un.tensor], (unsigned long long)cnt);
  }
}

__global__ __launch_bounds__(256) void counts_zero_kernel(unsigned long long* __restrict__ counts, int32_t n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) counts[i] = 0ull;
}

}  // namespace

bool apexw_q8_fast_eligible(uint32_t flags, uint32_t block) { return apexw_q8_fast_ok(flags, block); }

bool apexw_q8_flags_ok(uint32_t flags, uint32_t block, int64_t n) {
  const uint32_t pd = (flags >> APEXW_FLAG_PDT_SHIFT) & 3u, gd = (flags >> APEXW_FLAG_GDT_SHIFT) & 3u;
  if (!(pd == APEXW_F32 || pd == APEXW_BF16 || pd == APEXW_F16) || gd != pd) return false;
  const uint32_t md = (flags >> APEXW_FLAG_MDT_SHIFT) & 3u, vd = (flags >> APEXW_FLAG_VDT_SHIFT) & 3u;
  const uint32_t cd = pd == APEXW_F16 ? APEXW_F16 : APEXW_BF16;   // the parameter's compact dtype
  if (flags & APEXW_FLAG_DENSE) {
    // units of 2048 elements; fp32 m comes with fp32 v
    if (block != 2048 || (flags & (APEXW_FLAG_ULTRA | APEXW_FLAG_NF4 | APEXW_FLAG_QUAD))) return false;
    if (md == APEXW_F32) return vd == APEXW_F32;
    return md == cd && (vd == cd || vd == APEXW_F32);
  }
  if (block == 0 || block > 2048) return false;
  if (flags & APEXW_FLAG_ULTRA) {
    // INT8 m, dense v; a dense v needs no v scales
    if (flags & (APEXW_FLAG_NF4 | APEXW_FLAG_QUAD)) return false;
    if (!(vd == cd || vd == APEXW_F32)) return false;
    return (block % 8) == 0 || (flags & APEXW_FLAG_SCALAR);
  }
  if ((flags & APEXW_FLAG_QUAD) && (!(flags & APEXW_FLAG_NF4) || (block % 8) != 0 || (n % 4) != 0)) return false;
  if ((flags & APEXW_FLAG_NF4) && (block % 8) != 0) return false;
  if ((block % 8) != 0 && !(flags & APEXW_FLAG_SCALAR)) return false;
  return true;
}

int apexw_launch_q8(const apexw_tensor* tensors, int64_t n_units, const apexw_unit* units,
                    const apexw_hparams* hp, hipStream_t stream) {
  if (hp->mode == APEXW_MODE_SINGLE) {
    const int grid = apexw_resident_grid((const void*)q8_step_kernel<true>, n_units);
    hipLaunchKernelGGL(q8_step_kernel<true>, dim3(grid), dim3(256), 0, stream, tensors, units, n_units, *hp);
  } else {
    const int grid = apexw_resident_grid((const void*)q8_step_kernel<false>, n_units);
    hipLaunchKernelGGL(q8_step_kernel<false>, dim3(grid), dim3(256), 0, stream, tensors, units, n_units, *hp);
  }
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

int apexw_launch_q8_cautious_count(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units,
                                   int64_t n_units, const apexw_hparams* hp, hipStream_t stream) {
  // the counters are cleared by a kernel (not hipMemsetAsync), which a captured graph replays reliably
  hipLaunchKernelGGL(counts_zero_kernel, dim3((unsigned)((n_tensors + 255) / 256)), dim3(256), 0, stream, hp->counts,
                     n_tensors);
  if (n_units > 0) {
    const int grid = apexw_resident_grid((const void*)q8_cautious_count_kernel, n_units);
    hipLaunchKernelGGL(q8_cautious_count_kernel, dim3(grid), dim3(256), 0, stream, tensors, units, n_units, *hp);
  }
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

int apexw_launch_ultra(const apexw_tensor* tensors, int64_t n_units, const apexw_unit* units,
                       const apexw_hparams* hp, hipStream_t stream) {
  const int grid = apexw_resident_grid((const void*)ultra_step_kernel, n_units);
  hipLaunchKernelGGL(ultra_step_kernel, dim3(grid), dim3(256), 0, stream, tensors, units, n_units, *hp);
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

int apexw_launch_q8_fast(const apexw_tensor* tensors, int64_t n_units, const apexw_unit* units,
                         const apexw_hparams* hp, int32_t p_dtype, hipStream_t stream) {
  // one workgroup per kFastChunk units: the hardware dispatcher balances the tail
  // (measured ~1% faster than a persistent grid of 16 workgroups per resident slot)
  const int64_t chunks = (n_units + kFastChunk - 1) / kFastChunk;
  const int grid = (int)(chunks < INT32_MAX ? chunks : INT32_MAX);
  const bool sr = hp->flags & APEXW_HP_SR;
  const bool b1hi = !(hp->flags & APEXW_HP_LERP_HI) && (hp->flags & APEXW_HP_LOOK_HI);
#define APEXW_FAST(PD, SR, HI, GC) \
  hipLaunchKernelGGL((q8_fast_kernel<PD, SR, HI, GC>), dim3(grid), dim3(256), 0, stream, tensors, units, n_units, *hp)
  if (hp->rows) {
    // centralized tensors in the launch
    if (p_dtype == APEXW_F32) {
      if (sr) { if (b1hi) APEXW_FAST(APEXW_F32, true, true, true); else APEXW_FAST(APEXW_F32, true, false, true); }
      else { if (b1hi) APEXW_FAST(APEXW_F32, false, true, true); else APEXW_FAST(APEXW_F32, false, false, true); }
    } else {
      if (sr) { if (b1hi) APEXW_FAST(APEXW_BF16, true, true, true); else APEXW_FAST(APEXW_BF16, true, false, true); }
      else { if (b1hi) APEXW_FAST(APEXW_BF16, false, true, true); else APEXW_FAST(APEXW_BF16, false, false, true); }
    }
  } else if (p_dtype == APEXW_F32) {
    if (sr) { if (b1hi) APEXW_FAST(APEXW_F32, true, true, false); else APEXW_FAST(APEXW_F32, true, false, false); }
    else { if (b1hi) APEXW_FAST(APEXW_F32, false, true, false); else APEXW_FAST(APEXW_F32, false, false, false); }
  } else {
    if (sr) { if (b1hi) APEXW_FAST(APEXW_BF16, true, true, false); else APEXW_FAST(APEXW_BF16, true, false, false); }
    else { if (b1hi) APEXW_FAST(APEXW_BF16, false, true, false); else APEXW_FAST(APEXW_BF16, false, false, false); }
  }
#undef APEXW_FAST
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}
