// Factored second moment (row / column EMA of g^2) for large matrices, with an
// INT8, packed 6-bit or 16-bit first moment (gfx950).
//
// Restates the reference's _apply_factored_v_int8_update (apexw/state.py:442-608),
// which precision "8bit" (ApexW._step_ultra, apexw/optimizer.py:4380-4400) and
// "compact" (_multi_tensor_step, :5382-5432; plan replay, :1141-1163) call for
// tensors with is_factored_v.  Three launches per step cover every factored
// tensor of a group:
//
//  1. statistics: one workgroup per band of 32 rows.  A lane owns 8 adjacent
//     columns of a 2048-column pass; it sums the squares of its columns down the
//     band (column partials, written per band) and of its elements per row
//     (row partials, reduced across the workgroup at the end of the band).  The
//     grad is read once, in 4 KiB row segments per wave.
//  2. finalisation: column blocks of 256 sum the band partials (fp64) and apply
//     the column EMA; one workgroup per tensor applies the row EMA, reduces the
//     row mean and writes sqrt(row / mean) in place of the row sums.
//  3. update: one wave per unit (quantization block, or 2048 elements for 16-bit
//     m): den = max(row_norm[r] col_sqrt[c] + eps_scaled, eps), m lerp, p update,
//     block requantization with the EMA-max scale (0.9).
//
// The reductions sum in a different order than torch's CPU kernels, so the row
// and column EMAs agree with the reference to a few fp32 ulps, not bit for bit;
// everything after them is elementwise and follows the reference's op order.
#include "common.h"

namespace {

constexpr int kBand = APEXW_FV_BAND_ROWS;
constexpr int kPass = 2048;  // columns per statistics pass (256 lanes x 8)

struct FvCtx {
  const apexw_hparams* hp;
  float coef;
};

APEXW_DEV float unit_uniform(uint32_t r16) { return ((float)(r16 & 0xFFFFu) + 0.5f) * (1.0f / 65536.0f); }

APEXW_DEV float lerp_to(float a, float b, float coef, bool hi) {
  // torch lerp(a, b, w): |w| < 0.5 -> a + w*(b-a); else b + (w-1)*(b-a), one FMA each
  return hi ? fmaf(coef, b - a, b) : fmaf(coef, b - a, a);
}

// _prepare_grads (sanitize in the grad dtype when clipping; AMP unscale before a
// clip; clip), then _prep_grad_chunk_fp32 (apexw/state.py:261-280): nan_to_num in
// fp32 and the AMP unscale when no clip consumed it.
template <int GD> APEXW_DEV float fv_grad(float g, const FvCtx& c) {
  const apexw_hparams& hp = *c.hp;
  const bool unscale = hp.flags & APEXW_HP_UNSCALE, clip = hp.flags & APEXW_HP_CLIP;
  if (hp.flags & APEXW_HP_SANITIZE) g = sanitize<GD>(g);
  if (unscale && clip) g = rnd<GD>(g * hp.grad_inv_scale);
  if (clip) g = rnd<GD>(g * c.coef);
  if (hp.flags & APEXW_HP_FV_SANITIZE) {
    if (__builtin_isnan(g)) g = 0.0f;
    else if (__builtin_isinf(g)) g = g > 0.0f ? 65504.0f : -65504.0f;
  }
  if (unscale && !clip) g *= hp.grad_inv_scale;
  return g;
}

APEXW_DEV int fv_find_band(const apexw_fv_tensor* fv, int n_fv, int64_t band) {
  int lo = 0, hi = n_fv - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (fv[mid].band0 <= band) lo = mid; else hi = mid - 1;
  }
  return lo;
}

APEXW_DEV int fv_find_cb(const apexw_fv_tensor* fv, int n_fv, int64_t cb) {
  int lo = 0, hi = n_fv - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (fv[mid].cb0 <= cb) lo = mid; else hi = mid - 1;
  }
  return lo;
}

APEXW_DEV int fv_find_tensor(const apexw_fv_tensor* fv, int n_fv, uint32_t tensor) {
  int lo = 0, hi = n_fv - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (fv[mid].tensor <= tensor) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// workspace of one tensor: [rows] row sums, then row norms in place;
// [n_bands x cols] column partials; [cols] column square roots
struct FvWs {
  float* row;
  float* part;
  float* col;
};
APEXW_DEV FvWs fv_ws(float* ws, const apexw_fv_tensor& e) {
  const int64_t nb = (e.rows + kBand - 1) / kBand;
  float* base = ws + e.ws;
  return {base, base + e.rows, base + e.rows + nb * (int64_t)e.cols};
}

// ---------------------------------------------------------------------------
// 1. statistics
// ---------------------------------------------------------------------------
// band: the band's index within its tensor
template <int GD>
APEXW_DEV void fv_stats_band(const apexw_tensor& t, const apexw_fv_tensor& e, int64_t band, float* ws,
                             const FvCtx& c) {
  __shared__ float s_row[4][kBand];
  const FvWs w = fv_ws(ws, e);
  const int64_t cols = e.cols;
  const int r0 = (int)(band * kBand);
  const int nr = min(kBand, e.rows - r0);
  const bool vec = !(t.flags & APEXW_FLAG_SCALAR) && (cols % 8) == 0;
  float racc[kBand];
#pragma unroll
  for (int i = 0; i < kBand; ++i) racc[i] = 0.0f;
  for (int64_t c0 = 0; c0 < cols; c0 += kPass) {
    const int64_t cb = c0 + (int64_t)threadIdx.x * 8;
    const int cnt = cb >= cols ? 0 : (int)((cols - cb) < 8 ? (cols - cb) : 8);
    float cacc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) cacc[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < kBand; ++i) {
      if (i < nr && cnt > 0) {
        const int64_t e0 = (int64_t)(r0 + i) * cols + cb;
        float g[8];
        if (vec && cnt == 8) {
          load8<GD>(t.g, e0, g);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) g[j] = j < cnt ? load1<GD>(t.g, e0 + j) : 0.0f;
        }
        float rs = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x = j < cnt ? fv_grad<GD>(g[j], c) : 0.0f;
          const float sq = x * x;
          cacc[j] = cacc[j] + sq;
          rs = rs + sq;
        }
        racc[i] = racc[i] + rs;
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < cnt) w.part[band * cols + cb + j] = cacc[j];
  }
  // rows: reduce each row partial across the workgroup
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < kBand; ++i) {
    const float s = wave_sum(racc[i]);
    if (lane == 0) s_row[wave][i] = s;
  }
  __syncthreads();
  if ((int)threadIdx.x < nr) {
    const int i = threadIdx.x;
    w.row[r0 + i] = ((s_row[0][i] + s_row[1][i]) + s_row[2][i]) + s_row[3][i];
  }
}

__global__ __launch_bounds__(256) void fv_stats_kernel(const apexw_tensor* __restrict__ tensors,
                                                       const apexw_fv_tensor* __restrict__ fv, int n_fv,
                                                       float* __restrict__ ws, apexw_hparams hp) {
  const int64_t band = blockIdx.x;
  const int k = fv_find_band(fv, n_fv, band);
  const apexw_fv_tensor e = fv[k];
  const apexw_tensor& t = tensors[e.tensor];
  FvCtx c;
  c.hp = &hp;
  c.coef = (hp.flags & APEXW_HP_CLIP) ? *hp.clip_coef : 1.0f;
  const int64_t lb = band - e.band0;
  if (((t.flags >> APEXW_FLAG_GDT_SHIFT) & 3u) == APEXW_F32) fv_stats_band<APEXW_F32>(t, e, lb, ws, c);
  else fv_stats_band<APEXW_BF16>(t, e, lb, ws, c);
}

// ---------------------------------------------------------------------------
// 2. finalisation
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fv_finalize_kernel(const apexw_tensor* __restrict__ tensors,
                                                          const apexw_fv_tensor* __restrict__ fv, int n_fv,
                                                          int64_t n_col_blocks, float* __restrict__ ws,
                                                          apexw_hparams hp) {
  __shared__ double s_sum[4];
  const int64_t b = blockIdx.x;
  if (b < n_col_blocks) {
    // column EMA: the reference's mean over rows, or sum * (1-b2)/rows above 262,144 elements
    const int k = fv_find_cb(fv, n_fv, b);
    const apexw_fv_tensor e = fv[k];
    const apexw_tensor& t = tensors[e.tensor];
    const FvWs w = fv_ws(ws, e);
    const int64_t col = (b - e.cb0) * 256 + threadIdx.x;
    if (col >= e.cols) return;
    const int64_t nb = (e.rows + kBand - 1) / kBand;
    double s = 0.0;
    for (int64_t i = 0; i < nb; ++i) s += (double)w.part[i * e.cols + col];
    float* cv = t.v_scale;
    const float old = cv[col];
    float cn;
    if (e.flags & APEXW_FV_SUM_COLS) {
      cn = fmaf((float)s, hp.one_minus_beta2 / (float)e.rows, old * hp.beta2);
    } else {
      cn = fmaf((float)(s / (double)e.rows), hp.one_minus_beta2, old * hp.beta2);
    }
    if (!(fabsf(cn) <= 3.402823466e38f)) cn = 0.0f;  // nan_to_num(0, 0, 0)
    cv[col] = cn;
    w.col[col] = sqrtf(cn);
    return;
  }
  // rows: EMA, nan_to_num, mean over rows, sqrt(row / mean)
  const apexw_fv_tensor e = fv[b - n_col_blocks];
  const apexw_tensor& t = tensors[e.tensor];
  const FvWs w = fv_ws(ws, e);
  float* rv = (float*)t.v;
  double acc = 0.0;
  for (int r = threadIdx.x; r < e.rows; r += 256) {
    const float mean = (float)((double)w.row[r] / (double)e.cols);
    float rn = fmaf(mean, hp.one_minus_beta2, rv[r] * hp.beta2);
    if (!(fabsf(rn) <= 3.402823466e38f)) rn = 0.0f;
    rv[r] = rn;
    acc += (double)rn;
  }
  // workgroup sum in fp64
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) s_sum[threadIdx.x >> 6] = acc;
  __syncthreads();
  const double tot = ((s_sum[0] + s_sum[1]) + s_sum[2]) + s_sum[3];
  const float mean = fmaxf((float)(tot / (double)e.rows), 1e-30f);
  const float inv = 1.0f / mean;
  for (int r = threadIdx.x; r < e.rows; r += 256) w.row[r] = sqrtf(rv[r] * inv);
}

// ---------------------------------------------------------------------------
// 3. update
// ---------------------------------------------------------------------------
// m kinds
constexpr int kM8 = 0;    // INT8 codes
constexpr int kM6 = 1;    // packed 6-bit codes (code + 31, 4 codes per 3 bytes, little-endian 24-bit words)
constexpr int kM16 = 2;   // bf16 tensor

template <int PD, int MK>
APEXW_DEV void fv_unit(const apexw_tensor& t, const apexw_fv_tensor& e, uint32_t tix, uint32_t unit, float* ws,
                       const FvCtx& c) {
  constexpr int GD = PD;
  const apexw_hparams& hp = *c.hp;
  const bool sr = hp.flags & APEXW_HP_SR;
  const bool wd = t.flags & APEXW_FLAG_WD;
  const bool vec = !(t.flags & APEXW_FLAG_SCALAR);
  const FvWs w = fv_ws(ws, e);
  const int64_t bs = MK == kM16 ? APEXW_COMPACT_UNIT : (int64_t)t.block;
  const int64_t start = (int64_t)unit * bs;
  const int64_t cnt_unit = (t.n - start) < bs ? (t.n - start) : bs;
  const int lane = lane_id();
  const int64_t cols = e.cols;
  const float ms_old = MK == kM16 ? 0.0f : t.m_scale[unit];
  const uint32_t key = rng_key(hp.seed, tix, hp.step, 3u, (uint32_t)(start >> 32));

  float mnew[4][8];
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t rel = (int64_t)(k * 64 + lane) * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) mnew[k][j] = 0.0f;
    const int cnt = rel >= cnt_unit ? 0 : (int)((cnt_unit - rel) < 8 ? (cnt_unit - rel) : 8);
    if (cnt == 0) continue;
    const int64_t e0 = start + rel;
    const bool full = vec && cnt == 8;
    float p[8], g[8], m[8];
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
    if constexpr (MK == kM8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) m[j] = j < cnt ? (float)((const int8_t*)t.m)[e0 + j] * ms_old : 0.0f;
    } else if constexpr (MK == kM6) {
      // e0 is a multiple of 4 (blocks are multiples of 4): two 3-byte words
      const uint8_t* mb = (const uint8_t*)t.m + (e0 >> 2) * 3;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (4 * q < cnt) {
          const uint32_t wd24 = (uint32_t)mb[3 * q] | ((uint32_t)mb[3 * q + 1] << 8) | ((uint32_t)mb[3 * q + 2] << 16);
#pragma unroll
          for (int i = 0; i < 4; ++i) m[4 * q + i] = ((float)((wd24 >> (6 * i)) & 63u) - 31.0f) * ms_old;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) m[4 * q + i] = 0.0f;
        }
      }
    } else {
      if (full) {
        load8<APEXW_BF16>(t.m, e0, m);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) m[j] = j < cnt ? load1<APEXW_BF16>(t.m, e0 + j) : 0.0f;
      }
    }
    // row / column of element e0; later elements step across the row boundary
    int64_t row = e0 / cols;
    int64_t col = e0 - row * cols;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < cnt) {
        const float x = fv_grad<GD>(g[j], c);
        m[j] = lerp_to(m[j], x, hp.lerp_coef, hp.flags & APEXW_HP_LERP_HI);
        const float den = fmaxf(w.row[row] * w.col[col] + hp.eps_scaled, hp.eps);
        const float upd = (m[j] / den) * hp.step_size;
        if constexpr (PD == APEXW_F32) {
          p[j] = (wd ? p[j] * hp.wd_factor : p[j]) - upd;
        } else {
          const float pd = wd ? rnd<PD>(p[j] * hp.wd_factor) : p[j];
          p[j] = rnd<PD>(pd - rnd<PD>(upd));
        }
        mnew[k][j] = m[j];
        amax = fmaxf(amax, fabsf(m[j]));
        if (++col == cols) {
          col = 0;
          ++row;
        }
      }
    }
    if (full) {
      store8<PD>(t.p, e0, p);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < cnt) store1<PD>(t.p, e0 + j, p[j]);
    }
    if constexpr (MK == kM16) {
      if (full) {
        store8<APEXW_BF16>(t.m, e0, m);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (j < cnt) store1<APEXW_BF16>(t.m, e0 + j, m[j]);
      }
    }
  }
  if constexpr (MK == kM16) return;
  // ---- requantize m with the block absmax (EMA-max against the old scale)
  amax = wave_max(amax);
  float ms = fmaxf(amax, 1e-12f) / (MK == kM8 ? 127.0f : 31.0f);
  ms = fmaxf(ms, ms_old * 0.9f);
  if (lane == 0) t.m_scale[unit] = ms;
  const float lim = MK == kM8 ? 127.0f : 31.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t rel = (int64_t)(k * 64 + lane) * 8;
    const int cnt = rel >= cnt_unit ? 0 : (int)((cnt_unit - rel) < 8 ? (cnt_unit - rel) : 8);
    if (cnt == 0) continue;
    const int64_t e0 = start + rel;
    int32_t qc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float y = mnew[k][j] / ms;  // padding elements are 0 -> code 0
      if (sr) y = y + (unit_uniform(rng_at(key, (uint32_t)(e0 + j)) >> 16) - 0.5f);
      qc[j] = (int32_t)fminf(fmaxf(rintf(y), -lim), lim);
    }
    if constexpr (MK == kM8) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < cnt) ((int8_t*)t.m)[e0 + j] = (int8_t)qc[j];
    } else {
      uint8_t* mb = (uint8_t*)t.m + (e0 >> 2) * 3;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        // a quad wholly past the tensor's end is block padding and keeps code 31 (zero);
        // a partial quad writes code 31 in its padding slots
        if (4 * q < cnt) {
          uint32_t wd24 = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t u = (4 * q + i < cnt) ? (uint32_t)(qc[4 * q + i] + 31) : 31u;
            wd24 |= u << (6 * i);
          }
          mb[3 * q] = (uint8_t)(wd24 & 0xFFu);
          mb[3 * q + 1] = (uint8_t)((wd24 >> 8) & 0xFFu);
          mb[3 * q + 2] = (uint8_t)((wd24 >> 16) & 0xFFu);
        }
      }
    }
  }
}

__global__ __launch_bounds__(256) void fv_update_kernel(const apexw_tensor* __restrict__ tensors,
                                                        const apexw_fv_tensor* __restrict__ fv, int n_fv,
                                                        const apexw_unit* __restrict__ units, int64_t n_units,
                                                        float* __restrict__ ws, apexw_hparams hp) {
  FvCtx c;
  c.hp = &hp;
  c.coef = (hp.flags & APEXW_HP_CLIP) ? *hp.clip_coef : 1.0f;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const int64_t stride = (int64_t)gridDim.x * 4;
  for (int64_t u = (int64_t)blockIdx.x * 4 + wave; u < n_units; u += stride) {
    const apexw_unit un = units[u];
    const apexw_tensor& t = tensors[un.tensor];
    const apexw_fv_tensor& e = fv[fv_find_tensor(fv, n_fv, un.tensor)];
    if (e.tensor != un.tensor || !(t.flags & APEXW_FLAG_FACTORED)) continue;  // never taken for a valid plan
    const bool p32 = ((t.flags >> APEXW_FLAG_PDT_SHIFT) & 3u) == APEXW_F32;
    if (t.block == 0) {
      if (p32) fv_unit<APEXW_F32, kM16>(t, e, un.tensor, un.unit, ws, c);
      else fv_unit<APEXW_BF16, kM16>(t, e, un.tensor, un.unit, ws, c);
    } else if (t.flags & APEXW_FLAG_M6) {
      if (p32) fv_unit<APEXW_F32, kM6>(t, e, un.tensor, un.unit, ws, c);
      else fv_unit<APEXW_BF16, kM6>(t, e, un.tensor, un.unit, ws, c);
    } else {
      if (p32) fv_unit<APEXW_F32, kM8>(t, e, un.tensor, un.unit, ws, c);
      else fv_unit<APEXW_BF16, kM8>(t, e, un.tensor, un.unit, ws, c);
    }
  }
}

}  // namespace

int apexw_launch_factored(const apexw_tensor* tensors, const apexw_fv_tensor* fv, int32_t n_fv, int64_t n_bands,
                          int64_t n_col_blocks, const apexw_unit* units, int64_t n_units, float* ws,
                          const apexw_hparams* hp, hipStream_t stream) {
  hipLaunchKernelGGL(fv_stats_kernel, dim3((unsigned)n_bands), dim3(256), 0, stream, tensors, fv, n_fv, ws, *hp);
  hipLaunchKernelGGL(fv_finalize_kernel, dim3((unsigned)(n_col_blocks + n_fv)), dim3(256), 0, stream, tensors, fv,
                     n_fv, n_col_blocks, ws, *hp);
  if (n_units > 0) {
    const int grid = apexw_resident_grid((const void*)fv_update_kernel, n_units);
    hipLaunchKernelGGL(fv_update_kernel, dim3(grid), dim3(256), 0, stream, tensors, fv, n_fv, units, n_units, ws,
                       *hp);
  }
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}
