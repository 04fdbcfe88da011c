// Optimizer-state conversion between precision modes (gfx950).
//
// A checkpoint written by one precision mode (compact: 16/32-bit m and v;
// 8-bit: NF4 or INT8 m codes and log-uint8 v codes with per-block fp32 scales)
// is expanded to fp32 moments (apexw_state_decode) and rebuilt in another
// mode's layout (apexw_state_encode).  The quantizers are the reference's with
// no previous scale (apexw/quantization.py): INT8 scale = max(absmax, 1e-12) /
// 127, q = round(x / scale) clamped to +-127 (:66-126); NF4 scale =
// max(absmax, 1e-12), code = searchsorted(midpoints, clamp(x / scale, -1, 1))
// (ties to the lower code, pad nibble 7 for an odd count, :277-357); log-uint8
// vmax = max(block max, 1e-12), q = round(log2(max(v / vmax, 2^-24)) 254/24 +
// 255) clamped to [1, 255], 0 where v <= 0 (:381-448).  A quad-shared v
// (one value per 4 consecutive elements) decodes to its value on each of the 4
// and encodes as the mean of the 4, summed pairwise ((a + b) + (c + d)) / 4 so
// that 4 equal values give back exactly that value.  All roundings to nearest
// (even); the conversion runs once per load, so the kernels favour simplicity:
// one wave per unit (a quantization block, or 2048 elements of a dense state),
// elements strided over the lanes.
#include "common.h"
#include "luts.h"

namespace {

constexpr int kUnit = 2048;

struct Conv {
  apexw_state_layout s;
  int64_t n_units;
};

APEXW_DEV int64_t unit_len(const apexw_state_layout& s) {
  return s.kind == APEXW_STATE_Q8 ? (int64_t)s.block : (int64_t)kUnit;
}

template <int DT> APEXW_DEV float ld(const void* base, int64_t i) { return load1<DT>(base, i); }

APEXW_DEV float load_dense(const void* base, uint32_t dt, int64_t i) {
  if (dt == APEXW_F32) return ld<APEXW_F32>(base, i);
  if (dt == APEXW_BF16) return ld<APEXW_BF16>(base, i);
  return ld<APEXW_F16>(base, i);
}

APEXW_DEV void store_dense(void* base, uint32_t dt, int64_t i, float x) {
  if (dt == APEXW_F32) store1<APEXW_F32>(base, i, x);
  else if (dt == APEXW_BF16) store1<APEXW_BF16>(base, i, rnd<APEXW_BF16>(x));
  else store1<APEXW_F16>(base, i, rnd<APEXW_F16>(x));
}

// fp32 mean of a quad, pairwise
APEXW_DEV float quad_mean(const float* v, int64_t q) {
  const float a = v[4 * q], b = v[4 * q + 1], c = v[4 * q + 2], d = v[4 * q + 3];
  return ((a + b) + (c + d)) * 0.25f;
}

APEXW_DEV uint32_t nf4_nearest(float normed) {
  uint32_t code = 0;
#pragma unroll
  for (int k = 0; k < 14; ++k) {
    const float mid = (kNf4Code[k] + kNf4Code[k + 1]) * 0.5f;
    code += mid < normed ? 1u : 0u;
  }
  return code;
}

APEXW_DEV uint32_t logu8_nearest(float v, float vmax) {
  if (!(v > 0.0f)) return 0u;
  const float r = fmaxf(v / vmax, 0x1p-24f);
  const float q = rintf(log2f(r) * 0x1.52aaaap+3f + 255.0f);   // fp32(254/24)
  return (uint32_t)fminf(fmaxf(q, 1.0f), 255.0f);
}

__global__ __launch_bounds__(256) void decode_kernel(Conv c, float* __restrict__ m_out, float* __restrict__ v_out) {
  const apexw_state_layout& s = c.s;
  const int lane = lane_id();
  const int64_t len = unit_len(s);
  const uint32_t md = (s.flags >> APEXW_FLAG_MDT_SHIFT) & 3u, vd = (s.flags >> APEXW_FLAG_VDT_SHIFT) & 3u;
  const bool quad = s.flags & APEXW_FLAG_QUAD, nf4 = s.flags & APEXW_FLAG_NF4;
  for (int64_t u = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); u < c.n_units; u += (int64_t)gridDim.x * 4) {
    const int64_t e0 = u * len;
    const int64_t e1 = e0 + len < s.n ? e0 + len : s.n;
    if (s.kind == APEXW_STATE_Q8) {
      const float ms = s.m_scale[u], vs = s.v_scale[u];
      for (int64_t i = e0 + lane; i < e1; i += 64) {
        float m;
        if (nf4) {
          const uint32_t byte = APEXW_GLOBAL(const uint8_t, s.m)[i >> 1];
          m = kNf4Code[(i & 1) ? (byte & 15u) : (byte >> 4)] * ms;
        } else {
          m = (float)APEXW_GLOBAL(const int8_t, s.m)[i] * ms;
        }
        const uint32_t code = APEXW_GLOBAL(const uint8_t, s.v)[quad ? (i >> 2) : i];
        m_out[i] = m;
        v_out[i] = kVLogLut[code] * vs;
      }
    } else {
      for (int64_t i = e0 + lane; i < e1; i += 64) {
        m_out[i] = load_dense(s.m, md, i);
        v_out[i] = load_dense(s.v, vd, quad ? (i >> 2) : i);
      }
    }
  }
}

__global__ __launch_bounds__(256) void encode_kernel(Conv c, const float* __restrict__ m_in,
                                                     const float* __restrict__ v_in) {
  const apexw_state_layout& s = c.s;
  const int lane = lane_id();
  const int64_t len = unit_len(s);
  const uint32_t md = (s.flags >> APEXW_FLAG_MDT_SHIFT) & 3u, vd = (s.flags >> APEXW_FLAG_VDT_SHIFT) & 3u;
  const bool quad = s.flags & APEXW_FLAG_QUAD, nf4 = s.flags & APEXW_FLAG_NF4;
  for (int64_t u = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); u < c.n_units; u += (int64_t)gridDim.x * 4) {
    const int64_t e0 = u * len;
    const int64_t e1 = e0 + len < s.n ? e0 + len : s.n;
    if (s.kind != APEXW_STATE_Q8) {
      for (int64_t i = e0 + lane; i < e1; i += 64) store_dense(s.m, md, i, m_in[i]);
      if (quad) {
        for (int64_t q = (e0 >> 2) + lane; q < (e1 >> 2); q += 64) store_dense(s.v, vd, q, quad_mean(v_in, q));
      } else {
        for (int64_t i = e0 + lane; i < e1; i += 64) store_dense(s.v, vd, i, v_in[i]);
      }
      continue;
    }
    // block scales: m absmax, v max over the block's (quad) values, NaN -> 0
    float amax = 0.0f, vmax = 0.0f;
    for (int64_t i = e0 + lane; i < e1; i += 64) amax = fmaxf(amax, fabsf(m_in[i]));
    if (quad) {
      for (int64_t q = (e0 >> 2) + lane; q < (e1 >> 2); q += 64) {
        const float x = quad_mean(v_in, q);
        vmax = fmaxf(vmax, x > 3.402823466e38f ? 0.0f : x);   // fmaxf drops a NaN operand
      }
    } else {
      for (int64_t i = e0 + lane; i < e1; i += 64) {
        const float x = v_in[i];
        vmax = fmaxf(vmax, x > 3.402823466e38f ? 0.0f : x);
      }
    }
    amax = fmaxf(wave_max(amax), 1e-12f);
    vmax = fmaxf(wave_max(vmax), 1e-12f);
    const float ms = nf4 ? amax : amax / 127.0f;
    if (lane == 0) {
      s.m_scale[u] = ms;
      s.v_scale[u] = vmax;
    }
    if (nf4) {
      // one byte per lane per pass: elements 2b (high nibble) and 2b + 1 (low; pad 7 past the end)
      for (int64_t b = (e0 >> 1) + lane; b < ((e1 + 1) >> 1); b += 64) {
        const int64_t i = 2 * b;
        const uint32_t hi = nf4_nearest(fminf(fmaxf(m_in[i] / ms, -1.0f), 1.0f));
        const uint32_t lo = i + 1 < e1 ? nf4_nearest(fminf(fmaxf(m_in[i + 1] / ms, -1.0f), 1.0f)) : 7u;
        APEXW_GLOBAL(uint8_t, s.m)[b] = (uint8_t)((hi << 4) | lo);
      }
    } else {
      for (int64_t i = e0 + lane; i < e1; i += 64) {
        const float q = fminf(fmaxf(rintf(m_in[i] / ms), -127.0f), 127.0f);
        APEXW_GLOBAL(int8_t, s.m)[i] = (int8_t)q;
      }
    }
    if (quad) {
      for (int64_t q = (e0 >> 2) + lane; q < (e1 >> 2); q += 64) {
        const float x = quad_mean(v_in, q);
        APEXW_GLOBAL(uint8_t, s.v)[q] = (uint8_t)logu8_nearest(x > 3.402823466e38f ? 0.0f : x, vmax);
      }
    } else {
      for (int64_t i = e0 + lane; i < e1; i += 64) {
        const float x = v_in[i];
        APEXW_GLOBAL(uint8_t, s.v)[i] = (uint8_t)logu8_nearest(x > 3.402823466e38f ? 0.0f : x, vmax);
      }
    }
  }
}

int check(const apexw_state_layout* s) {
  if (!s || !s->m || !s->v || s->n <= 0 || s->reserved != 0) return APEXW_ERR_ARG;
  const uint32_t f = s->flags;
  const bool quad = f & APEXW_FLAG_QUAD;
  if (quad && (s->n % 4) != 0) return APEXW_ERR_ARG;
  if (s->kind == APEXW_STATE_Q8) {
    if (!s->m_scale || !s->v_scale) return APEXW_ERR_ARG;
    if (s->block == 0 || s->block > 2048) return APEXW_ERR_ARG;
    if ((quad || (f & APEXW_FLAG_NF4)) && (s->block % 8) != 0) return APEXW_ERR_ARG;
    if (f & ~(APEXW_FLAG_QUAD | APEXW_FLAG_NF4)) return APEXW_ERR_ARG;
  } else if (s->kind == APEXW_STATE_DENSE) {
    const uint32_t md = (f >> APEXW_FLAG_MDT_SHIFT) & 3u, vd = (f >> APEXW_FLAG_VDT_SHIFT) & 3u;
    if (md > APEXW_F16 || vd > APEXW_F16) return APEXW_ERR_DTYPE;
    if (f & ~(APEXW_FLAG_QUAD | (3u << APEXW_FLAG_MDT_SHIFT) | (3u << APEXW_FLAG_VDT_SHIFT))) return APEXW_ERR_ARG;
    if (s->block != 0) return APEXW_ERR_ARG;
  } else {
    return APEXW_ERR_ARG;
  }
  return APEXW_OK;
}

int launch(const apexw_state_layout* s, const float* a, const float* b, bool encode, void* stream) {
  const int st = check(s);
  if (st != APEXW_OK) return st;
  if (!a || !b) return APEXW_ERR_ARG;
  Conv c;
  c.s = *s;
  const int64_t len = s->kind == APEXW_STATE_Q8 ? (int64_t)s->block : (int64_t)kUnit;
  c.n_units = (s->n + len - 1) / len;
  const int64_t wg = (c.n_units + 3) / 4;
  const int grid = (int)(wg < 65536 ? wg : 65536);
  hipStream_t hs = (hipStream_t)stream;
  if (encode)
    hipLaunchKernelGGL(encode_kernel, dim3(grid), dim3(256), 0, hs, c, a, b);
  else
    hipLaunchKernelGGL(decode_kernel, dim3(grid), dim3(256), 0, hs, c, (float*)a, (float*)b);
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

}  // namespace

extern "C" int apexw_state_decode(const apexw_state_layout* s, float* m_out, float* v_out, void* stream) {
  return launch(s, m_out, v_out, false, stream);
}

extern "C" int apexw_state_encode(const apexw_state_layout* s, const float* m_in, const float* v_in, void* stream) {
  return launch(s, m_in, v_in, true, stream);
}
