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
//     At the end of the band it applies the row EMA to the band's rows and
//     keeps their sum.
//  2. finalisation: column blocks of 64 sum the band partials (fp64) and apply
//     the column EMA; one workgroup per tensor sums the band sums into the row
//     mean.
//  3. update: one wave per unit (quantization block, or 2048 elements for 16-bit
//     m): den = max(sqrt(row[r] / mean) col_sqrt[c] + eps_scaled, eps), m lerp,
//     p update, block requantization with the EMA-max scale (0.9).
//
// The reductions sum in a different order than torch's CPU kernels, so the row
// and column EMAs agree with the reference to a few fp32 ulps, not bit for bit;
// everything after them is elementwise and follows the reference's op order.
#include "common.h"

namespace {

constexpr int kBand = APEXW_FV_BAND_ROWS;
constexpr int kPass = 2048;  // columns per statistics pass (256 lanes x 8)
constexpr int kColBlock = 64;  // columns per finalisation workgroup

struct FvCtx {
  const apexw_hparams* hp;
  float coef;
};

APEXW_DEV float unit_uniform(uint32_t r16) { return ((float)(r16 & 0xFFFFu) + 0.5f) * (1.0f / 65536.0f); }

// Division with a refined reciprocal and one FMA residual correction (Markstein):
// equal to the IEEE quotient except within ~2^-46 of a rounding midpoint.  The
// divisors here are positive, finite and normal (scales >= 1e-12 / 127,
// denominators >= eps).
APEXW_DEV float rcp_refined(float y) {
  const float r0 = __builtin_amdgcn_rcpf(y);
  return fmaf(fmaf(-y, r0, 1.0f), r0, r0);
}
APEXW_DEV float div_refined(float x, float y, float r) {
  const float q0 = x * r;
  return fmaf(fmaf(-q0, y, x), r, q0);
}

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

// fv_grad as selects on the launch-uniform flags: no per-element branches in
// the unrolled single-row update.  Same values as fv_grad.
template <int GD> APEXW_DEV float fv_grad_sel(float g, const FvCtx& c) {
  const uint32_t f = c.hp->flags;
  const bool unscale = f & APEXW_HP_UNSCALE, clip = f & APEXW_HP_CLIP;
  const float big = rnd<GD>(65504.0f);
  float x = g;
  const float xs = __builtin_isnan(x) ? 0.0f : (__builtin_isinf(x) ? __builtin_copysignf(big, x) : x);
  x = (f & APEXW_HP_SANITIZE) ? xs : x;
  const float xu = rnd<GD>(x * c.hp->grad_inv_scale);
  x = (unscale && clip) ? xu : x;
  const float xc = rnd<GD>(x * c.coef);
  x = clip ? xc : x;
  const float xf = __builtin_isnan(x) ? 0.0f : (__builtin_isinf(x) ? __builtin_copysignf(65504.0f, x) : x);
  x = (f & APEXW_HP_FV_SANITIZE) ? xf : x;
  return (unscale && !clip) ? x * c.hp->grad_inv_scale : x;
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

// workspace of one tensor: aux = [n_bands] band sums of the new row EMA, then
// the inverse row mean at aux[n_bands]; [n_bands x cols] column partials;
// [cols] column square roots
struct FvWs {
  float* aux;
  float* part;
  float* col;
};
APEXW_DEV int64_t fv_round4(int64_t x) { return (x + 3) & ~(int64_t)3; }
APEXW_DEV FvWs fv_ws(float* ws, const apexw_fv_tensor& e) {
  // each part starts on a 16-byte boundary (apexw_factored_layout sizes them the same way)
  const int64_t nb = (e.rows + kBand - 1) / kBand;
  float* base = ws + e.ws;
  float* part = base + fv_round4(nb + 1);
  return {base, part, part + fv_round4(nb * (int64_t)e.cols)};
}

// ---------------------------------------------------------------------------
// 1. statistics
// ---------------------------------------------------------------------------
// band: the band's index within its tensor.  Writes the band's column partials,
// applies the row EMA to its rows (exp_avg_sq_row) and leaves the band's sum of
// the new row values in aux[band] for the row mean.
// g^2 of one grad element.  PLAIN: no grad-dtype sanitize, clip or AMP unscale,
// only the fp32 nan_to_num (NaN -> 0, +-inf -> +-65504), as selects.
template <int GD, bool PLAIN> APEXW_DEV float fv_sq(float g, const FvCtx& c, bool fv_sanitize) {
  if constexpr (PLAIN) {
    const float sq = g * g;
    if (!fv_sanitize) return sq;
    return __builtin_isnan(g) ? 0.0f : (__builtin_isinf(g) ? 65504.0f * 65504.0f : sq);
  } else {
    const float x = fv_grad<GD>(g, c);
    return x * x;
  }
}

// band: the band's index within its tensor.  Writes the band's column partials,
// applies the row EMA to its rows (exp_avg_sq_row) and leaves the band's sum of
// the new row values in aux[band] for the row mean.
//
// A pass whose 32 x 2048 tile lies inside the tensor (and PLAIN) loads its rows
// in batches (128 bytes per lane); other passes go row by row.  Both keep the
// row partials in registers and sum in the same order, so the statistics do not
// depend on which path a pass took.
template <int GD, bool PLAIN>
APEXW_DEV void fv_stats_band(const apexw_tensor& t, const apexw_fv_tensor& e, int64_t band, float* ws,
                             const FvCtx& c, float (*s_row)[kBand], float (*s_t)[kBand][65]) {
  const FvWs w = fv_ws(ws, e);
  const apexw_hparams& hp = *c.hp;
  const bool fs = hp.flags & APEXW_HP_FV_SANITIZE;
  const int64_t cols = e.cols;
  const int r0 = (int)(band * kBand);
  const int nr = min(kBand, e.rows - r0);
  const bool vec = !(t.flags & APEXW_FLAG_SCALAR) && (cols % 8) == 0;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float racc[kBand];
#pragma unroll
  for (int i = 0; i < kBand; ++i) racc[i] = 0.0f;
  for (int64_t c0 = 0; c0 < cols; c0 += kPass) {
    const int64_t cb = c0 + (int64_t)threadIdx.x * 8;
    const int cnt = cb >= cols ? 0 : (int)((cols - cb) < 8 ? (cols - cb) : 8);
    float cacc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) cacc[j] = 0.0f;
    if (PLAIN && vec && nr == kBand && c0 + kPass <= cols) {
      constexpr int B = GD == APEXW_F32 ? 4 : 8;  // rows per batch: 128 bytes per lane
#pragma unroll
      for (int i0 = 0; i0 < kBand; i0 += B) {
        float g[B][8];
#pragma unroll
        for (int i = 0; i < B; ++i) load8<GD>(t.g, (int64_t)(r0 + i0 + i) * cols + cb, g[i]);
#pragma unroll
        for (int i = 0; i < B; ++i) {
          float rs = 0.0f;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float sq = fv_sq<GD, PLAIN>(g[i][j], c, fs);
            cacc[j] = cacc[j] + sq;
            rs = rs + sq;
          }
          racc[i0 + i] = racc[i0 + i] + rs;
        }
      }
    } else {
      // row by row; the same summation order as the whole-tile path (per lane:
      // the row's 8 squares, then across passes; per column: down the rows)
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
            const float sq = j < cnt ? fv_sq<GD, PLAIN>(g[j], c, fs) : 0.0f;
            cacc[j] = cacc[j] + sq;
            rs = rs + sq;
          }
          racc[i] = racc[i] + rs;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < cnt) w.part[band * cols + cb + j] = cacc[j];
  }
  // rows: the register row partials go through LDS transposed (row-major with a
  // 65-float stride, conflict-free both ways); lane r < 32 of each wave sums its
  // row over the wave's 64 lanes in lane order, then the waves' sums are combined
  // and the row EMA applied
#pragma unroll
  for (int i = 0; i < kBand; ++i) s_t[wave][i][lane] = racc[i];
  __syncthreads();
  if (lane < kBand) {
    float rsum = 0.0f;
#pragma unroll 16
    for (int l = 0; l < 64; ++l) rsum += s_t[wave][lane][l];
    s_row[wave][lane] = rsum;
  }
  __syncthreads();
  if (wave == 0) {
    float rn = 0.0f;
    if (lane < nr) {
      const float sum = ((s_row[0][lane] + s_row[1][lane]) + s_row[2][lane]) + s_row[3][lane];
      const float mean = (float)((double)sum / (double)cols);
      float* rv = (float*)t.v;
      rn = fmaf(mean, hp.one_minus_beta2, rv[r0 + lane] * hp.beta2);
      if (!(fabsf(rn) <= 3.402823466e38f)) rn = 0.0f;  // nan_to_num(0, 0, 0)
      rv[r0 + lane] = rn;
    }
    const float bs = wave_sum(rn);
    if (lane == 0) w.aux[band] = bs;
  }
}

// PLAIN (no grad-dtype sanitize, clip or AMP unscale) is a launch-wide property:
// one instantiation each, so the plain kernel keeps its own register budget.
template <bool PLAIN>
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
  // one copy of the LDS for both grad dtypes' instantiations
  __shared__ float s_row[4][kBand];
  __shared__ float s_t[4][kBand][65];
  const uint32_t gdt = (t.flags >> APEXW_FLAG_GDT_SHIFT) & 3u;
  if (gdt == APEXW_F32) fv_stats_band<APEXW_F32, PLAIN>(t, e, lb, ws, c, s_row, s_t);
  else if (gdt == APEXW_F16) fv_stats_band<APEXW_F16, PLAIN>(t, e, lb, ws, c, s_row, s_t);
  else fv_stats_band<APEXW_BF16, PLAIN>(t, e, lb, ws, c, s_row, s_t);
}

// ---------------------------------------------------------------------------
// 2. finalisation
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fv_finalize_kernel(const apexw_tensor* __restrict__ tensors,
                                                          const apexw_fv_tensor* __restrict__ fv, int n_fv,
                                                          int64_t n_col_blocks, float* __restrict__ ws,
                                                          apexw_hparams hp) {
  __shared__ double s_sum[4];
  __shared__ double s_col[4][kColBlock];
  const int64_t b = blockIdx.x;
  if (b < n_col_blocks) {
    // column EMA: the reference's mean over rows, or sum * (1-b2)/rows above 262,144 elements.
    // 64 columns per workgroup, each summed by 4 waves over interleaved bands
    // (4 fp64 accumulators per lane), then combined in a fixed order.
    const int k = fv_find_cb(fv, n_fv, b);
    const apexw_fv_tensor e = fv[k];
    const apexw_tensor& t = tensors[e.tensor];
    const FvWs w = fv_ws(ws, e);
    const int slice = threadIdx.x >> 6;
    const int64_t col = (b - e.cb0) * kColBlock + (threadIdx.x & 63);
    const int64_t nb = (e.rows + kBand - 1) / kBand;
    if (col < e.cols) {
      double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
      int64_t i = slice;
      for (; i + 12 < nb; i += 16) {
        a0 += (double)w.part[i * e.cols + col];
        a1 += (double)w.part[(i + 4) * e.cols + col];
        a2 += (double)w.part[(i + 8) * e.cols + col];
        a3 += (double)w.part[(i + 12) * e.cols + col];
      }
      for (; i < nb; i += 4) a0 += (double)w.part[i * e.cols + col];
      s_col[slice][threadIdx.x & 63] = (a0 + a1) + (a2 + a3);
    }
    __syncthreads();
    if (slice != 0 || col >= e.cols) return;
    const int l = threadIdx.x & 63;
    const double s = ((s_col[0][l] + s_col[1][l]) + s_col[2][l]) + s_col[3][l];
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
  // rows: mean of the new row EMA (band sums in fp64) -> 1 / max(mean, 1e-30)
  const apexw_fv_tensor e = fv[b - n_col_blocks];
  const FvWs w = fv_ws(ws, e);
  const int64_t nb = (e.rows + kBand - 1) / kBand;
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < nb; i += 256) acc += (double)w.aux[i];
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) s_sum[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    const double tot = ((s_sum[0] + s_sum[1]) + s_sum[2]) + s_sum[3];
    const float mean = fmaxf((float)(tot / (double)e.rows), 1e-30f);
    w.aux[nb] = 1.0f / mean;
  }
}

// ---------------------------------------------------------------------------
// 3. update
// ---------------------------------------------------------------------------
// m kinds
constexpr int kM8 = 0;    // INT8 codes
constexpr int kM6 = 1;    // packed 6-bit codes (code + 31, 4 codes per 3 bytes, little-endian 24-bit words)
constexpr int kM16 = 2;   // 16-bit tensor: fp16 for fp16 parameters, else bf16

template <int PD, int MK>
APEXW_DEV void fv_unit(const apexw_tensor& t, const apexw_fv_tensor& e, uint32_t tix, uint32_t unit, float* ws,
                       const FvCtx& c) {
  constexpr int GD = PD;
  constexpr int MD16 = PD == APEXW_F16 ? APEXW_F16 : APEXW_BF16;
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
  // row factor sqrt(row / mean(row)), as the reference forms it per row
  const float* rvec = (const float*)t.v;
  const float inv = w.aux[(e.rows + kBand - 1) / kBand];

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
        load8<MD16>(t.m, e0, m);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) m[j] = j < cnt ? load1<MD16>(t.m, e0 + j) : 0.0f;
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
        const float den = fmaxf(sqrtf(rvec[row] * inv) * w.col[col] + hp.eps_scaled, hp.eps);
        const float upd = (m[j] / den) * hp.step_size;
        if constexpr (PD == APEXW_F32) {
          p[j] = (wd ? p[j] * hp.wd_factor : p[j]) - upd;
        } else if constexpr (PD == APEXW_F16) {
          // p.float(), mul_(wd), sub_(update), clamp_(-65504, 65504) (NaN kept), one rounding
          const float pf = (wd ? p[j] * hp.wd_factor : p[j]) - upd;
          p[j] = rnd<PD>(pf > 65504.0f ? 65504.0f : (pf < -65504.0f ? -65504.0f : pf));
        } else {
          const float pd = wd ? rnd<PD>(p[j] * hp.wd_factor) : p[j];
          p[j] = rnd<PD>(pd - rnd<PD>(upd));
        }
        mnew[k][j] = m[j];
        amax = fmaxf(amax, fabsf(m[j]));
        if constexpr (MK == kM16) m[j] = rnd<MD16>(m[j]);  // m.copy_(mf.to(m.dtype)): nearest-even
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
        store8<MD16>(t.m, e0, m);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (j < cnt) store1<MD16>(t.m, e0 + j, m[j]);
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

// SR noise for two elements from one xorshift32 step: the two 16-bit halves,
// each as (h + 0.5) / 65536 - 0.5, uniform and symmetric on (-0.5, 0.5).
APEXW_DEV void sr_pair(uint32_t& rs, float& n0, float& n1) {
  rs ^= rs << 13;
  rs ^= rs >> 17;
  rs ^= rs << 5;
  constexpr float k = 1.0f / 65536.0f, o = 0.5f / 65536.0f - 0.5f;
  n0 = fmaf((float)(rs & 0xFFFFu), k, o);
  n1 = fmaf((float)(rs >> 16), k, o);
}

// A whole 2048-element unit with 16-byte aligned buffers: every load of the wave
// is issued before any arithmetic, m moves as 8-byte (INT8) / 6-byte (6-bit) /
// 16-byte (bf16) vectors, and the row / column of each lane's first element
// comes from one 32-bit division per group.  Same arithmetic as fv_unit.
template <int PD, int MK>
APEXW_DEV void fv_unit_full(const apexw_tensor& t, const apexw_fv_tensor& e, uint32_t tix, uint32_t unit,
                            float* ws, const FvCtx& c) {
  constexpr int GD = PD;
  constexpr int W = PD == APEXW_F32 ? 2 : 1;  // 16-byte words per 8 elements of p / g
  const apexw_hparams& hp = *c.hp;
  const bool sr = hp.flags & APEXW_HP_SR;
  const bool wd = t.flags & APEXW_FLAG_WD;
  const FvWs w = fv_ws(ws, e);
  const int64_t start = (int64_t)unit * 2048;
  const int lane = lane_id();
  const uint32_t cols = (uint32_t)e.cols;
  const int64_t row0 = start / (int64_t)cols;
  const uint32_t col0 = (uint32_t)(start - row0 * (int64_t)cols);
  const float ms_old = MK == kM16 ? 0.0f : t.m_scale[unit];
  const uint32_t key = rng_key(hp.seed, tix, hp.step, 3u, (uint32_t)(start >> 32));
  const float* rvec = (const float*)t.v;
  const float inv = w.aux[(e.rows + kBand - 1) / kBand];
  // ---- loads
  u32x4 praw[4][W], graw[4][W];
  u32x4 mw16[MK == kM16 ? 4 : 1];
  u32x2 mw8[MK == kM16 ? 1 : 4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t e0 = start + k * 512 + lane * 8;
    const auto pp = APEXW_GLOBAL(const u32x4, (const uint8_t*)t.p + e0 * (PD == APEXW_F32 ? 4 : 2));
    const auto gp = APEXW_GLOBAL(const u32x4, (const uint8_t*)t.g + e0 * (GD == APEXW_F32 ? 4 : 2));
#pragma unroll
    for (int i = 0; i < W; ++i) {
      praw[k][i] = __builtin_nontemporal_load(pp + i);
      graw[k][i] = __builtin_nontemporal_load(gp + i);
    }
    if constexpr (MK == kM16) {
      mw16[k] = __builtin_nontemporal_load(APEXW_GLOBAL(const u32x4, (const uint16_t*)t.m + e0));
    } else if constexpr (MK == kM8) {
      mw8[k] = __builtin_nontemporal_load(APEXW_GLOBAL(const u32x2, (const int8_t*)t.m + e0));
    } else {
      // 6 bytes at (e0 / 4) * 3, 2-byte aligned: three 16-bit words
      const auto mp = APEXW_GLOBAL(const uint16_t, (const uint8_t*)t.m + (e0 >> 2) * 3);
      const uint32_t h0 = mp[0], h1 = mp[1], h2 = mp[2];
      mw8[k] = u32x2{h0 | ((h1 & 0xFFu) << 16), (h1 >> 8) | (h2 << 8)};
    }
  }
  // ---- update
  float mnew[4][8];
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t e0 = start + k * 512 + lane * 8;
    float p[8], g[8], m[8];
    const uint32_t* pw = (const uint32_t*)&praw[k][0];
    const uint32_t* gw = (const uint32_t*)&graw[k][0];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = PD == APEXW_F32 ? __uint_as_float(pw[j]) : (j & 1 ? __uint_as_float(pw[j >> 1] & 0xFFFF0000u)
                                                              : bf16_bits_to_f32(pw[j >> 1] & 0xFFFFu));
      g[j] = GD == APEXW_F32 ? __uint_as_float(gw[j]) : (j & 1 ? __uint_as_float(gw[j >> 1] & 0xFFFF0000u)
                                                              : bf16_bits_to_f32(gw[j >> 1] & 0xFFFFu));
    }
    if constexpr (MK == kM16) {
      const uint32_t* mw = (const uint32_t*)&mw16[k];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        m[j] = j & 1 ? __uint_as_float(mw[j >> 1] & 0xFFFF0000u) : bf16_bits_to_f32(mw[j >> 1] & 0xFFFFu);
    } else if constexpr (MK == kM8) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        m[j] = (float)(int8_t)(((j < 4 ? mw8[k].x : mw8[k].y) >> (8 * (j & 3))) & 0xFFu) * ms_old;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        m[j] = ((float)(((j < 4 ? mw8[k].x : mw8[k].y) >> (6 * (j & 3))) & 63u) - 31.0f) * ms_old;
    }
    uint32_t x = col0 + (uint32_t)(k * 512 + lane * 8);
    const uint32_t rq = x / cols;
    int64_t row = row0 + rq;
    uint32_t col = x - rq * cols;
    float den[8];
    if (col + 8 <= cols) {
      // the 8 elements share a row: one row factor, the column roots as two 16-byte loads when aligned
      const float rv = sqrtf(rvec[row] * inv);
      float cs[8];
      if ((col & 3u) == 0) {
        const float4 a = *(const float4*)(w.col + col), b = *(const float4*)(w.col + col + 4);
        cs[0] = a.x; cs[1] = a.y; cs[2] = a.z; cs[3] = a.w; cs[4] = b.x; cs[5] = b.y; cs[6] = b.z; cs[7] = b.w;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) cs[j] = w.col[col + j];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) den[j] = fmaxf(rv * cs[j] + hp.eps_scaled, hp.eps);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        den[j] = fmaxf(sqrtf(rvec[row] * inv) * w.col[col] + hp.eps_scaled, hp.eps);
        if (++col == cols) {
          col = 0;
          ++row;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float gj = fv_grad<GD>(g[j], c);
      m[j] = lerp_to(m[j], gj, hp.lerp_coef, hp.flags & APEXW_HP_LERP_HI);
      const float upd = div_refined(m[j], den[j], rcp_refined(den[j])) * hp.step_size;
      if constexpr (PD == APEXW_F32) {
        p[j] = (wd ? p[j] * hp.wd_factor : p[j]) - upd;
      } else {
        const float pd = wd ? rnd<PD>(p[j] * hp.wd_factor) : p[j];
        p[j] = rnd<PD>(pd - rnd<PD>(upd));
      }
      mnew[k][j] = m[j];
      amax = fmaxf(amax, fabsf(m[j]));
      if constexpr (MK == kM16) m[j] = rnd<APEXW_BF16>(m[j]);  // m.copy_(mf.to(bf16)): nearest-even
    }
    store8<PD>(t.p, e0, p);
    if constexpr (MK == kM16) store8<APEXW_BF16>(t.m, e0, m);
  }
  if constexpr (MK == kM16) return;
  // ---- requantize m
  amax = wave_max(amax);
  float ms = fmaxf(amax, 1e-12f) / (MK == kM8 ? 127.0f : 31.0f);
  ms = fmaxf(ms, ms_old * 0.9f);
  if (lane == 0) t.m_scale[unit] = ms;
  const float lim = MK == kM8 ? 127.0f : 31.0f;
  const float rms = rcp_refined(ms);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t e0 = start + k * 512 + lane * 8;
    float y[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = div_refined(mnew[k][j], ms, rms);
    if (sr) {
      // SR noise: a per-lane xorshift32 stream seeded from the element index
      uint32_t rs = rng_at(key, (uint32_t)e0) | 1u;
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        float n0, n1;
        sr_pair(rs, n0, n1);
        y[j] = y[j] + n0;
        y[j + 1] = y[j + 1] + n1;
      }
    }
    uint32_t q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int32_t qi = (int32_t)fminf(fmaxf(rintf(y[j]), -lim), lim);
      q[j] = MK == kM8 ? ((uint32_t)qi & 0xFFu) : (uint32_t)(qi + 31);
    }
    if constexpr (MK == kM8) {
      const u32x2 v = {q[0] | (q[1] << 8) | (q[2] << 16) | (q[3] << 24), q[4] | (q[5] << 8) | (q[6] << 16) | (q[7] << 24)};
      __builtin_nontemporal_store(v, APEXW_GLOBAL(u32x2, (int8_t*)t.m + e0));
    } else {
      const uint32_t w0 = q[0] | (q[1] << 6) | (q[2] << 12) | (q[3] << 18);
      const uint32_t w1 = q[4] | (q[5] << 6) | (q[6] << 12) | (q[7] << 18);
      const auto mp = APEXW_GLOBAL(uint16_t, (uint8_t*)t.m + (e0 >> 2) * 3);
      mp[0] = (uint16_t)(w0 & 0xFFFFu);
      mp[1] = (uint16_t)((w0 >> 16) | ((w1 & 0xFFu) << 8));
      mp[2] = (uint16_t)(w1 >> 8);
    }
  }
}

// A whole unit inside one row of the matrix (cols % 4 == 0).  PLAIN: no grad-dtype
// sanitize / clip / AMP unscale and a lerp weight below 0.5; otherwise the grad
// goes through fv_grad_sel and the lerp picks its form per launch.  The row factor is one value for the unit and the column roots
// are 16-byte loads; the update's division is the refined one of fv_unit, and
// bf16 roundings convert pairs.  Returns false, before any load, when the unit
// crosses a row: the caller then runs fv_unit_full on it.
template <int PD, int MK, bool PLAIN>
APEXW_DEV bool fv_unit_row(const apexw_tensor& t, const apexw_fv_tensor& e, uint32_t tix, uint32_t unit,
                           float* ws, const FvCtx& c) {
  constexpr int W = PD == APEXW_F32 ? 2 : 1;  // 16-byte words per 8 elements of p / g
  const apexw_hparams& hp = *c.hp;
  const int64_t start = (int64_t)unit * 2048;
  const int64_t cols = e.cols;
  const int64_t row = start / cols;
  const uint32_t col0 = (uint32_t)(start - row * cols);
  if ((int64_t)col0 + 2048 > cols) return false;
  const FvWs w = fv_ws(ws, e);
  const int lane = lane_id();
  const bool sr = hp.flags & APEXW_HP_SR;
  const bool wd = t.flags & APEXW_FLAG_WD;
  const float ms_old = MK == kM16 ? 0.0f : t.m_scale[unit];
  // ---- loads
  u32x4 praw[4][W], graw[4][W];
  u32x4 mw16[MK == kM16 ? 4 : 1];
  u32x2 mw8[MK == kM16 ? 1 : 4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t e0 = start + k * 512 + lane * 8;
    const auto pp = APEXW_GLOBAL(const u32x4, (const uint8_t*)t.p + e0 * (PD == APEXW_F32 ? 4 : 2));
    const auto gp = APEXW_GLOBAL(const u32x4, (const uint8_t*)t.g + e0 * (PD == APEXW_F32 ? 4 : 2));
#pragma unroll
    for (int i = 0; i < W; ++i) {
      praw[k][i] = __builtin_nontemporal_load(pp + i);
      graw[k][i] = __builtin_nontemporal_load(gp + i);
    }
    if constexpr (MK == kM16) {
      mw16[k] = __builtin_nontemporal_load(APEXW_GLOBAL(const u32x4, (const uint16_t*)t.m + e0));
    } else if constexpr (MK == kM8) {
      mw8[k] = __builtin_nontemporal_load(APEXW_GLOBAL(const u32x2, (const int8_t*)t.m + e0));
    } else {
      const auto mp = APEXW_GLOBAL(const uint16_t, (const uint8_t*)t.m + (e0 >> 2) * 3);
      const uint32_t h0 = mp[0], h1 = mp[1], h2 = mp[2];
      mw8[k] = u32x2{h0 | ((h1 & 0xFFu) << 16), (h1 >> 8) | (h2 << 8)};
    }
  }
  const float rv = sqrtf(APEXW_GLOBAL(const float, t.v)[row] * APEXW_GLOBAL(const float, w.aux)[(e.rows + kBand - 1) / kBand]);
  // ---- grads; a non-finite grad (g * 0 is NaN exactly for inf / NaN) takes
  // the nan_to_num of _prep_grad_chunk_fp32 in registers (rare, wave-uniform branch)
  float g[4][8];
  float chk = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t* gw = (const uint32_t*)&graw[k][0];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      g[k][j] = PD == APEXW_F32 ? __uint_as_float(gw[j])
                                : (j & 1 ? __uint_as_float(gw[j >> 1] & 0xFFFF0000u) : __uint_as_float(gw[j >> 1] << 16));
      if constexpr (PLAIN) chk = fmaf(g[k][j], 0.0f, chk);
      else g[k][j] = fv_grad_sel<PD>(g[k][j], c);
    }
  }
  if (PLAIN && (hp.flags & APEXW_HP_FV_SANITIZE) && __builtin_amdgcn_ballot_w64(!(chk == 0.0f)) != 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float x = g[k][j];
        g[k][j] = __builtin_isnan(x) ? 0.0f : (__builtin_isinf(x) ? (x > 0.0f ? 65504.0f : -65504.0f) : x);
      }
  }
  // ---- update
  float mnew[MK == kM16 ? 1 : 4][8];
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t e0 = start + k * 512 + lane * 8;
    const uint32_t* pw = (const uint32_t*)&praw[k][0];
    float p[8], m[8], cs[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      p[j] = PD == APEXW_F32 ? __uint_as_float(pw[j])
                             : (j & 1 ? __uint_as_float(pw[j >> 1] & 0xFFFF0000u) : __uint_as_float(pw[j >> 1] << 16));
    if constexpr (MK == kM16) {
      const uint32_t* mw = (const uint32_t*)&mw16[k];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        m[j] = j & 1 ? __uint_as_float(mw[j >> 1] & 0xFFFF0000u) : __uint_as_float(mw[j >> 1] << 16);
    } else if constexpr (MK == kM8) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        m[j] = (float)(int8_t)(((j < 4 ? mw8[k].x : mw8[k].y) >> (8 * (j & 3))) & 0xFFu) * ms_old;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        m[j] = ((float)(((j < 4 ? mw8[k].x : mw8[k].y) >> (6 * (j & 3))) & 63u) - 31.0f) * ms_old;
    }
    {
      const auto cp = APEXW_GLOBAL(const u32x4, w.col + col0 + k * 512 + lane * 8);
      const u32x4 a = cp[0], b = cp[1];
      cs[0] = __uint_as_float(a.x); cs[1] = __uint_as_float(a.y); cs[2] = __uint_as_float(a.z);
      cs[3] = __uint_as_float(a.w); cs[4] = __uint_as_float(b.x); cs[5] = __uint_as_float(b.y);
      cs[6] = __uint_as_float(b.z); cs[7] = __uint_as_float(b.w);
    }
    float upd[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      m[j] = PLAIN ? fmaf(hp.lerp_coef, g[k][j] - m[j], m[j])
                   : lerp_to(m[j], g[k][j], hp.lerp_coef, hp.flags & APEXW_HP_LERP_HI);
      const float den = fmaxf(rv * cs[j] + hp.eps_scaled, hp.eps);
      upd[j] = div_refined(m[j], den, rcp_refined(den)) * hp.step_size;
      if constexpr (MK != kM16) {
        mnew[k][j] = m[j];
        amax = fmaxf(amax, fabsf(m[j]));
      }
    }
    const auto pp = APEXW_GLOBAL(u32x4, (uint8_t*)t.p + e0 * (PD == APEXW_F32 ? 4 : 2));
    if constexpr (PD == APEXW_F32) {
#pragma unroll
      for (int j = 0; j < 8; ++j) p[j] = (wd ? p[j] * hp.wd_factor : p[j]) - upd[j];
      __builtin_nontemporal_store(u32x4{__float_as_uint(p[0]), __float_as_uint(p[1]), __float_as_uint(p[2]),
                                        __float_as_uint(p[3])}, pp);
      __builtin_nontemporal_store(u32x4{__float_as_uint(p[4]), __float_as_uint(p[5]), __float_as_uint(p[6]),
                                        __float_as_uint(p[7])}, pp + 1);
    } else {
      // pairs: rnd(rnd(p * wd) - rnd(upd)), each rounding one packed conversion
      uint32_t out[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t pdw = wd ? pack_bf16x2(p[2 * i] * hp.wd_factor, p[2 * i + 1] * hp.wd_factor) : pw[i];
        const uint32_t uw = pack_bf16x2(upd[2 * i], upd[2 * i + 1]);
        out[i] = pack_bf16x2(__uint_as_float(pdw << 16) - __uint_as_float(uw << 16),
                             __uint_as_float(pdw & 0xFFFF0000u) - __uint_as_float(uw & 0xFFFF0000u));
      }
      __builtin_nontemporal_store(u32x4{out[0], out[1], out[2], out[3]}, pp);
    }
    if constexpr (MK == kM16) {
      // m.copy_(mf.to(bf16)): nearest-even
      const u32x4 mv = {pack_bf16x2(m[0], m[1]), pack_bf16x2(m[2], m[3]), pack_bf16x2(m[4], m[5]),
                        pack_bf16x2(m[6], m[7])};
      __builtin_nontemporal_store(mv, APEXW_GLOBAL(u32x4, (uint16_t*)t.m + e0));
    }
  }
  if constexpr (MK == kM16) {
    return true;
  } else {
    // ---- requantize m
    amax = wave_max(amax);
    constexpr float lim = MK == kM8 ? 127.0f : 31.0f;
    float ms = fmaxf(amax, 1e-12f) / lim;
    ms = fmaxf(ms, ms_old * 0.9f);
    if (lane == 0) t.m_scale[unit] = ms;
    const float rms = rcp_refined(ms);
    const uint32_t key = rng_key(hp.seed, tix, hp.step, 3u, (uint32_t)(start >> 32));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int64_t e0 = start + k * 512 + lane * 8;
      float y[8];
      if (sr) {
        // floor(m / scale + u), u = (h + 0.5) / 65536 from 16 random bits h: the
        // quotient as one product (the noise makes its last-ulp rounding immaterial)
        uint32_t rs = rng_at(key, (uint32_t)e0) | 1u;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          rs ^= rs << 13;
          rs ^= rs >> 17;
          rs ^= rs << 5;
          constexpr float k16 = 1.0f / 65536.0f, half = 0.5f / 65536.0f;
          y[j] = floorf(fmaf((float)(rs & 0xFFFFu), k16, fmaf(mnew[k][j], rms, half)));
          y[j + 1] = floorf(fmaf((float)(rs >> 16), k16, fmaf(mnew[k][j + 1], rms, half)));
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = rintf(div_refined(mnew[k][j], ms, rms));
      }
      uint32_t q[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int32_t qi = (int32_t)fminf(fmaxf(y[j], -lim), lim);
        q[j] = MK == kM8 ? ((uint32_t)qi & 0xFFu) : (uint32_t)(qi + 31);
      }
      if constexpr (MK == kM8) {
        const u32x2 v = {q[0] | (q[1] << 8) | (q[2] << 16) | (q[3] << 24), q[4] | (q[5] << 8) | (q[6] << 16) | (q[7] << 24)};
        __builtin_nontemporal_store(v, APEXW_GLOBAL(u32x2, (int8_t*)t.m + e0));
      } else {
        const uint32_t w0 = q[0] | (q[1] << 6) | (q[2] << 12) | (q[3] << 18);
        const uint32_t w1 = q[4] | (q[5] << 6) | (q[6] << 12) | (q[7] << 18);
        const auto mp = APEXW_GLOBAL(uint16_t, (uint8_t*)t.m + (e0 >> 2) * 3);
        mp[0] = (uint16_t)(w0 & 0xFFFFu);
        mp[1] = (uint16_t)((w0 >> 16) | ((w1 & 0xFFu) << 8));
        mp[2] = (uint16_t)(w1 >> 8);
      }
    }
    return true;
  }
}

// One kernel per (parameter dtype, m kind, PLAIN), each over its own range of
// units: no variant's register footprint lowers another's occupancy.
template <int PDK, int MK, bool PLAIN>
__global__ __launch_bounds__(256) void fv_update_kernel(const apexw_tensor* __restrict__ tensors,
                                                        const apexw_fv_tensor* __restrict__ fv, int n_fv,
                                                        const apexw_unit* __restrict__ units, int64_t n_units,
                                                        float* __restrict__ ws, apexw_hparams hp) {
  FvCtx c;
  c.hp = &hp;
  c.coef = (hp.flags & APEXW_HP_CLIP) ? *hp.clip_coef : 1.0f;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const int64_t stride = (int64_t)gridDim.x * 4;
  int64_t u = (int64_t)blockIdx.x * 4 + wave;
  // the next unit's descriptor is requested while this unit is processed
  apexw_unit next = u < n_units ? units[u] : apexw_unit{0u, 0u};
  for (; u < n_units; u += stride) {
    const apexw_unit un = next;
    if (u + stride < n_units) next = units[u + stride];
    // the checks below are never taken for a valid plan
    if (un.tensor >= (uint32_t)n_fv) continue;
    const apexw_fv_tensor& e = fv[un.tensor];
    const apexw_tensor& t = tensors[e.tensor];
    if (!(t.flags & APEXW_FLAG_FACTORED)) continue;
    const uint32_t pdt = (t.flags >> APEXW_FLAG_PDT_SHIFT) & 3u;
    const int mk = t.block == 0 ? kM16 : (t.flags & APEXW_FLAG_M6) ? kM6 : kM8;
    if (pdt != (uint32_t)PDK || mk != MK) continue;
    if constexpr (PDK == APEXW_F16) {
      // fp16 parameters take the general path (the full-unit and row paths unpack bf16 / fp32 words)
      fv_unit<PDK, MK>(t, e, e.tensor, un.unit, ws, c);
      continue;
    }
    const bool full = !(t.flags & APEXW_FLAG_SCALAR) && (t.block == 0 || t.block == 2048) &&
                      (int64_t)(un.unit + 1) * 2048 <= t.n;
    if (full) {
      if ((e.cols & 3) == 0 && fv_unit_row<PDK, MK, PLAIN>(t, e, e.tensor, un.unit, ws, c)) continue;
      fv_unit_full<PDK, MK>(t, e, e.tensor, un.unit, ws, c);
    } else {
      fv_unit<PDK, MK>(t, e, e.tensor, un.unit, ws, c);
    }
  }
}

template <int PDK, int MK>
void launch_update(const apexw_tensor* tensors, const apexw_fv_tensor* fv, int32_t n_fv, const apexw_unit* units,
                   int64_t begin, int64_t end, float* ws, const apexw_hparams* hp, hipStream_t stream) {
  if (end <= begin) return;
  const bool plain = !(hp->flags & (APEXW_HP_SANITIZE | APEXW_HP_CLIP | APEXW_HP_UNSCALE | APEXW_HP_LERP_HI));
  const void* fn = plain ? (const void*)fv_update_kernel<PDK, MK, true> : (const void*)fv_update_kernel<PDK, MK, false>;
  const int grid = apexw_resident_grid(fn, end - begin);
  if (plain)
    hipLaunchKernelGGL((fv_update_kernel<PDK, MK, true>), dim3(grid), dim3(256), 0, stream, tensors, fv, n_fv,
                       units + begin, end - begin, ws, *hp);
  else
    hipLaunchKernelGGL((fv_update_kernel<PDK, MK, false>), dim3(grid), dim3(256), 0, stream, tensors, fv, n_fv,
                       units + begin, end - begin, ws, *hp);
}

}  // namespace

int apexw_launch_factored(const apexw_tensor* tensors, const apexw_fv_tensor* fv, int32_t n_fv, int64_t n_bands,
                          int64_t n_col_blocks, const apexw_unit* units, const int64_t* ends, float* ws,
                          const apexw_hparams* hp, hipStream_t stream) {
  if (!(hp->flags & (APEXW_HP_SANITIZE | APEXW_HP_CLIP | APEXW_HP_UNSCALE)))
    hipLaunchKernelGGL(fv_stats_kernel<true>, dim3((unsigned)n_bands), dim3(256), 0, stream, tensors, fv, n_fv, ws, *hp);
  else
    hipLaunchKernelGGL(fv_stats_kernel<false>, dim3((unsigned)n_bands), dim3(256), 0, stream, tensors, fv, n_fv, ws, *hp);
  hipLaunchKernelGGL(fv_finalize_kernel, dim3((unsigned)(n_col_blocks + n_fv)), dim3(256), 0, stream, tensors, fv,
                     n_fv, n_col_blocks, ws, *hp);
  launch_update<APEXW_BF16, kM8>(tensors, fv, n_fv, units, 0, ends[0], ws, hp, stream);
  launch_update<APEXW_BF16, kM6>(tensors, fv, n_fv, units, ends[0], ends[1], ws, hp, stream);
  launch_update<APEXW_BF16, kM16>(tensors, fv, n_fv, units, ends[1], ends[2], ws, hp, stream);
  launch_update<APEXW_F32, kM8>(tensors, fv, n_fv, units, ends[2], ends[3], ws, hp, stream);
  launch_update<APEXW_F32, kM6>(tensors, fv, n_fv, units, ends[3], ends[4], ws, hp, stream);
  launch_update<APEXW_F32, kM16>(tensors, fv, n_fv, units, ends[4], ends[5], ws, hp, stream);
  launch_update<APEXW_F16, kM8>(tensors, fv, n_fv, units, ends[5], ends[6], ws, hp, stream);
  launch_update<APEXW_F16, kM6>(tensors, fv, n_fv, units, ends[6], ends[7], ws, hp, stream);
  launch_update<APEXW_F16, kM16>(tensors, fv, n_fv, units, ends[7], ends[8], ws, hp, stream);
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}
