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

namespace {

constexpr int kWaves = 4;

struct Q8Ctx {
  const apexw_hparams* hp;
  const float* vlut;   // LDS
  const float* code;   // LDS
  float coef;
};

APEXW_DEV float lerp_to(float a, float b, float coef, bool hi) {
  // torch lerp(a, b, w): |w| < 0.5 -> a + w*(b-a); else b + (w-1)*(b-a), one FMA each
  return hi ? fmaf(coef, b - a, b) : fmaf(coef, b - a, a);
}

// NF4 nearest code: searchsorted(mids, x) over the 14 decision points, using the
// symmetry mids[13-k] = -mids[k].
APEXW_DEV uint32_t nf4_rne(float x) {
  const float mids[7] = {APEXW_NF4_MIDS};
  const float a = fabsf(x);
  uint32_t lt = 0, le = 0;
#pragma unroll
  for (int k = 0; k < 7; ++k) {
    lt += (mids[k] < a) ? 1u : 0u;
    le += (mids[k] <= a) ? 1u : 0u;
  }
  return x >= 0.0f ? 7u + lt : 7u - le;
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

template <int GD> APEXW_DEV float q8_grad(float g, uint32_t tflags, const Q8Ctx& c) {
  const apexw_hparams& hp = *c.hp;
  if (hp.flags & APEXW_HP_SANITIZE) g = sanitize<GD>(g);
  if (hp.flags & APEXW_HP_CLIP) g = rnd<GD>(g * c.coef);
  // nan_to_num inside the step: on the fp32 copy (chunked) or on the grad dtype (generic)
  if (__builtin_isnan(g)) return 0.0f;
  if (__builtin_isinf(g)) {
    const float big = (tflags & (APEXW_FLAG_GENERIC | APEXW_FLAG_DENSE16)) ? rnd<GD>(65504.0f) : 65504.0f;
    return g > 0.0f ? big : -big;
  }
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
  return sr ? sr_round<PD>(x, r) : rnd<PD>(x);
}

// One quantization block per wavefront.
template <int PD, bool NF4, bool QUAD>
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
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      h[j] = sr ? rng_at(key, (uint32_t)(e0 + j)) : 0u;
      g[j] = q8_grad<GD>(g[j], tflags, c);
      m[j] = lerp_to(m[j], g[j], hp.lerp_coef, hp.flags & APEXW_HP_LERP_HI);
    }
    float num[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float look = lerp_to(g[j], m[j], hp.look_coef, hp.flags & APEXW_HP_LOOK_HI);
      num[j] = look * ((m[j] * g[j] >= 0.0f) ? hp.gain_hi : hp.gain_lo);
    }
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
        if (!(fabsf(vf) <= 3.402823466e38f)) vf = 0.0f;
        v[j] = vf;
        const float den = fmaxf(sqrtf(vf) + hp.eps_scaled, hp.eps);
        upd[j] = (num[j] / den) * hp.step_size;
      }
    }
    if constexpr (PD == APEXW_F32) {
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
  ms = fmaxf(ms, ms_old * 0.9f);
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
        mc[j] = sr ? nf4_sr(x, unit_uniform(r), c.code) : nf4_rne(x);
      } else {
        float y = mnew[k][j] / ms;
        if (sr) y = y + (unit_uniform(r) - 0.5f);
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

// Tensors under 64 elements in 8-bit mode keep 16-bit m/v (optimizer.py:4688-4735).
template <int PD, int VD>
APEXW_DEV void q8_dense16(const apexw_tensor& t, const Q8Ctx& c) {
  constexpr int GD = PD;
  const apexw_hparams& hp = *c.hp;
  const int lane = lane_id();
  if (lane >= t.n) return;
  const int64_t i = lane;
  float p = load1<PD>(t.p, i);
  float g = q8_grad<GD>(load1<GD>(t.g, i), t.flags, c);
  if (t.flags & APEXW_FLAG_WD) p = rnd<PD>(p * hp.wd_factor);
  const float mf = lerp_to(load1<APEXW_BF16>(t.m, i), g, hp.lerp_coef, hp.flags & APEXW_HP_LERP_HI);
  store1<APEXW_BF16>(t.m, i, rnd<APEXW_BF16>(mf));
  const float vf = fmaf(hp.one_minus_beta2 * g, g, load1<VD>(t.v, i) * hp.beta2);
  store1<VD>(t.v, i, rnd<VD>(vf));
  const float den = sqrtf(vf) + hp.eps_scaled;
  const float upd = (mf / den) * hp.step_size;
  if constexpr (PD == APEXW_F32) p = p - upd;
  else p = rnd<PD>(p - rnd<PD>(upd));
  store1<PD>(t.p, i, p);
}

__global__ __launch_bounds__(256) void q8_step_kernel(const apexw_tensor* __restrict__ tensors,
                                                      const apexw_unit* __restrict__ units,
                                                      int64_t n_units, apexw_hparams hp) {
  __shared__ float s_vlut[256];
  __shared__ float s_code[16];
  s_vlut[threadIdx.x] = kVLogLut[threadIdx.x];
  if (threadIdx.x < 16) s_code[threadIdx.x] = kNf4Code[threadIdx.x];
  __syncthreads();
  Q8Ctx c;
  c.hp = &hp;
  c.vlut = s_vlut;
  c.code = s_code;
  c.coef = (hp.flags & APEXW_HP_CLIP) ? *hp.clip_coef : 1.0f;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const int64_t stride = (int64_t)gridDim.x * kWaves;
  for (int64_t u = (int64_t)blockIdx.x * kWaves + wave; u < n_units; u += stride) {
    const apexw_unit un = units[u];
    const apexw_tensor& t = tensors[un.tensor];
    const uint32_t f = t.flags;
    const uint32_t pd = (f >> APEXW_FLAG_PDT_SHIFT) & 3u;
    if (f & APEXW_FLAG_DENSE16) {
      const uint32_t vd = (f >> APEXW_FLAG_VDT_SHIFT) & 3u;
      if (pd == APEXW_F32) {
        if (vd == APEXW_F32) q8_dense16<APEXW_F32, APEXW_F32>(t, c);
        else q8_dense16<APEXW_F32, APEXW_BF16>(t, c);
      } else {
        if (vd == APEXW_F32) q8_dense16<APEXW_BF16, APEXW_F32>(t, c);
        else q8_dense16<APEXW_BF16, APEXW_BF16>(t, c);
      }
      continue;
    }
    const bool nf4 = f & APEXW_FLAG_NF4, quad = f & APEXW_FLAG_QUAD;
    if (pd == APEXW_F32) {
      if (nf4 && quad) q8_block<APEXW_F32, true, true>(t, un.tensor, un.unit, c);
      else if (nf4) q8_block<APEXW_F32, true, false>(t, un.tensor, un.unit, c);
      else q8_block<APEXW_F32, false, false>(t, un.tensor, un.unit, c);
    } else {
      if (nf4 && quad) q8_block<APEXW_BF16, true, true>(t, un.tensor, un.unit, c);
      else if (nf4) q8_block<APEXW_BF16, true, false>(t, un.tensor, un.unit, c);
      else q8_block<APEXW_BF16, false, false>(t, un.tensor, un.unit, c);
    }
  }
}

}  // namespace

bool apexw_q8_flags_ok(uint32_t flags, uint32_t block, int64_t n) {
  const uint32_t pd = (flags >> APEXW_FLAG_PDT_SHIFT) & 3u, gd = (flags >> APEXW_FLAG_GDT_SHIFT) & 3u;
  if (!(pd == APEXW_F32 || pd == APEXW_BF16) || gd != pd) return false;
  if (flags & APEXW_FLAG_DENSE16) {
    const uint32_t md = (flags >> APEXW_FLAG_MDT_SHIFT) & 3u, vd = (flags >> APEXW_FLAG_VDT_SHIFT) & 3u;
    return n <= 64 && md == APEXW_BF16 && (vd == APEXW_BF16 || vd == APEXW_F32);
  }
  if (block == 0 || block > 2048) return false;
  if ((flags & APEXW_FLAG_QUAD) && (!(flags & APEXW_FLAG_NF4) || (block % 8) != 0 || (n % 4) != 0)) return false;
  if ((flags & APEXW_FLAG_NF4) && (block % 8) != 0) return false;
  if ((block % 8) != 0 && !(flags & APEXW_FLAG_SCALAR)) return false;
  return true;
}

int apexw_launch_q8(const apexw_tensor* tensors, int64_t n_units, const apexw_unit* units,
                    const apexw_hparams* hp, int grid, hipStream_t stream) {
  hipLaunchKernelGGL(q8_step_kernel, dim3(grid), dim3(256), 0, stream, tensors, units, n_units, *hp);
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}
