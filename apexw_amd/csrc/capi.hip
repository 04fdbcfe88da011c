// C-ABI entry points of libapexw_hip.so (declared in include/apexw_hip.h).
//
// Each entry point checks its scalar arguments before enqueueing anything and
// returns an apexw_status.  Tensor and unit tables are device-resident arrays
// built once per execution plan by the caller; apexw_check_tensor validates one
// descriptor (host copy) when the plan is built, so the per-step calls do not
// copy or inspect the tables.
#include <algorithm>
#include <mutex>
#include <queue>
#include <vector>

#include "common.h"

int apexw_launch_compact(const apexw_tensor*, int64_t, const apexw_unit*, const apexw_hparams*, hipStream_t);
int apexw_launch_q8(const apexw_tensor*, int64_t, const apexw_unit*, const apexw_hparams*, hipStream_t);
int apexw_launch_q8_fast(const apexw_tensor*, int64_t, const apexw_unit*, const apexw_hparams*, int32_t, hipStream_t);
int apexw_launch_ultra(const apexw_tensor*, int64_t, const apexw_unit*, const apexw_hparams*, hipStream_t);
int apexw_launch_q8_cautious_count(const apexw_tensor*, int32_t, const apexw_unit*, int64_t, const apexw_hparams*,
                                   hipStream_t);
int apexw_launch_compact_cautious_count(const apexw_tensor*, int32_t, const apexw_unit*, int64_t,
                                        const apexw_hparams*, hipStream_t);
bool apexw_q8_fast_eligible(uint32_t flags, uint32_t block);
int apexw_launch_clip(const apexw_tensor*, int32_t, const apexw_unit*, int64_t, int64_t, const int64_t*, float*, float*,
                      float, float, uint32_t, float*, const apexw_amp_dyn*, const apexw_row_means*, hipStream_t);
int apexw_launch_amp_prepare(const float*, const float*, int32_t*, int32_t, const apexw_amp_launch*, int32_t,
                             apexw_amp_dyn*, hipStream_t);
bool apexw_compact_flags_ok(uint32_t flags);
int apexw_launch_gemm_nt(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, uint16_t*, int32_t, int32_t,
                         int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, int64_t, int64_t, int64_t,
                         int64_t, int64_t, float, float, hipStream_t);
int apexw_muon_partials(int64_t n);
int apexw_launch_muon_coordwise(float*, const void*, int32_t, void*, int32_t, int64_t, float, float, int32_t, float,
                                float, int32_t, float, const apexw_amp_dyn*, hipStream_t);
int apexw_launch_grad_prep(const apexw_grad_prep*, const apexw_unit*, int64_t, float, uint32_t, const apexw_amp_dyn*,
                           hipStream_t);
int apexw_launch_row_means(const apexw_grad_prep*, const apexw_unit*, int64_t, float, uint32_t, const apexw_amp_dyn*,
                           hipStream_t);
int apexw_launch_gemm_grouped(const apexw_gemm_problem*, const uint32_t*, const int32_t*, int32_t, int32_t,
                              const apexw_amp_dyn*, hipStream_t);
int apexw_launch_muon_prepare(float*, const void*, int32_t, int64_t, int64_t, float, float, int32_t, float, float,
                              uint16_t*, uint16_t*, int64_t, int64_t, bool, float*, const apexw_amp_dyn*, hipStream_t);
int apexw_launch_muon_apply(void*, int32_t, const uint16_t*, int64_t, int64_t, int64_t, bool, int32_t, float, int32_t,
                            float, const apexw_amp_dyn*, hipStream_t);
bool apexw_q8_flags_ok(uint32_t flags, uint32_t block, int64_t n);
int apexw_launch_factored(const apexw_tensor*, const apexw_fv_tensor*, int32_t, int64_t, int64_t, const apexw_unit*,
                          const int64_t*, float*, const apexw_hparams*, hipStream_t);

namespace {

constexpr int kMaxDevices = 64;
int g_cu_count[kMaxDevices];
std::once_flag g_cu_once[kMaxDevices];

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  std::call_once(g_cu_once[dev], [dev] {
    int cu = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0) cu = 256;
    g_cu_count[dev] = cu;
  });
  return g_cu_count[dev];
}

// Resident 256-thread workgroups per CU, cached per (device, kernel).
struct OccEntry {
  int dev;
  const void* kernel;
  int blocks;
};
constexpr int kMaxOcc = 64;
OccEntry g_occ[kMaxOcc];
int g_n_occ = 0;
std::mutex g_occ_mu;

int blocks_per_cu(const void* kernel) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  std::lock_guard<std::mutex> lk(g_occ_mu);
  for (int i = 0; i < g_n_occ; ++i)
    if (g_occ[i].dev == dev && g_occ[i].kernel == kernel) return g_occ[i].blocks;
  int b = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, kernel, 256, 0) != hipSuccess || b <= 0) b = 1;
  if (g_n_occ < kMaxOcc) g_occ[g_n_occ++] = {dev, kernel, b};
  return b;
}

bool hp_ok(const apexw_hparams* hp) {
  if (!hp) return false;
  if (hp->mode > APEXW_MODE_SINGLE) return false;
  // the per-parameter in-backward update uses the grads as given
  if (hp->mode == APEXW_MODE_SINGLE && (hp->flags & (APEXW_HP_SANITIZE | APEXW_HP_CLIP | APEXW_HP_UNSCALE)))
    return false;
  if ((hp->flags & APEXW_HP_CLIP) && !hp->clip_coef) return false;
  if ((hp->flags & APEXW_HP_CAUTIOUS) && (!hp->counts || hp->mode == APEXW_MODE_SINGLE)) return false;
  if ((hp->flags & APEXW_HP_AMSGRAD) && (!hp->max_v || ((uintptr_t)hp->max_v & 7u) || hp->mode == APEXW_MODE_SINGLE))
    return false;
  if ((hp->flags & APEXW_HP_SLOW) && (!hp->slow || ((uintptr_t)hp->slow & 7u) || hp->mode == APEXW_MODE_SINGLE))
    return false;
  if (hp->flags & APEXW_HP_AMP) {
    // device-side AMP scalars: the compact and 8-bit step modes, with the unscale they carry
    if (!hp->amp || ((uintptr_t)hp->amp & 15u) || hp->mode == APEXW_MODE_SINGLE) return false;
    if (!(hp->flags & APEXW_HP_UNSCALE)) return false;
  } else if ((hp->flags & APEXW_HP_UNSCALE) && !apexw_inv_scale_ok(hp->grad_inv_scale)) {
    return false;
  }
  return true;
}

}  // namespace

int apexw_resident_grid(const void* kernel, int64_t n_units) {
  const int64_t want = (n_units + 3) / 4;
  // 16 workgroups per resident slot: workgroups queue behind the resident ones,
  // so CUs that finish early pick up more of the grid (measured on the 8B 8-bit
  // step: 16x is ~4% faster than a grid of exactly the resident workgroups)
  const int64_t cap = (int64_t)cu_count() * blocks_per_cu(kernel) * 16;
  const int64_t g = want < cap ? want : cap;
  return (int)(g > 0 ? g : 1);
}

extern "C" {

int apexw_abi_version(void) { return APEXW_ABI_VERSION; }

// Validate one tensor descriptor (host memory) for the given step kind
// (0 = compact, 1 = 8-bit).  Returns APEXW_OK or the reason it is unsupported.
int apexw_check_tensor(const apexw_tensor* t, int32_t kind) {
  if (!t || !t->p || !t->g || !t->m || !t->v || t->n <= 0) return APEXW_ERR_ARG;
  // folded centralization: compact (row means in m_scale / block) and 8-bit / ultra
  // (row means in the launch's side table) steps; not the per-parameter or factored ones
  if ((t->flags & APEXW_FLAG_GC) && (kind == 3 || kind == 4)) return APEXW_ERR_ARG;
  if (kind == 0 || kind == 3) {
    if (!apexw_compact_flags_ok(t->flags)) return APEXW_ERR_DTYPE;
    // the per-parameter update takes grads in the parameter's dtype only
    if (kind == 3 && ((t->flags >> APEXW_FLAG_GDT_SHIFT) & 3u) != ((t->flags >> APEXW_FLAG_PDT_SHIFT) & 3u))
      return APEXW_ERR_DTYPE;
    if ((t->flags & APEXW_FLAG_QUAD) && (kind == 3 || (t->n % 4) != 0)) return APEXW_ERR_ARG;
    if ((t->flags & APEXW_FLAG_GC) && (!t->m_scale || t->block == 0 || (t->n % t->block) != 0)) return APEXW_ERR_ARG;
    if ((t->flags & APEXW_FLAG_VSCALE) && (!t->v_scale || ((uintptr_t)t->v_scale & 7u))) return APEXW_ERR_ARG;
  } else if (kind == 4) {
    // factored row: v / v_scale are the fp32 row / column EMAs
    const uint32_t f = t->flags;
    const uint32_t pd = (f >> APEXW_FLAG_PDT_SHIFT) & 3u, gd = (f >> APEXW_FLAG_GDT_SHIFT) & 3u;
    if (!(f & APEXW_FLAG_FACTORED) || !(pd == APEXW_F32 || pd == APEXW_BF16 || pd == APEXW_F16) || gd != pd)
      return APEXW_ERR_DTYPE;
    if (f & (APEXW_FLAG_QUAD | APEXW_FLAG_NF4 | APEXW_FLAG_DENSE)) return APEXW_ERR_ARG;
    if (t->block == 0) {
      // 16-bit m in the parameter's compact dtype: fp16 for fp16 parameters, else bf16
      const uint32_t md16 = pd == APEXW_F16 ? APEXW_F16 : APEXW_BF16;
      if ((f & APEXW_FLAG_M6) || ((f >> APEXW_FLAG_MDT_SHIFT) & 3u) != md16) return APEXW_ERR_DTYPE;
    } else {
      if (t->block > 2048 || !t->m_scale) return APEXW_ERR_ARG;
      if ((f & APEXW_FLAG_M6) && (t->block % 4) != 0) return APEXW_ERR_ARG;
    }
  } else if (kind == 1 || kind == 2 || kind == 5) {
    if (!apexw_q8_flags_ok(t->flags, t->block, t->n)) return APEXW_ERR_DTYPE;
    // kind 5: the ultra step's rows (INT8-m blocks or dense m / v); kind 1: never ultra rows
    if (kind == 5 && !(t->flags & (APEXW_FLAG_ULTRA | APEXW_FLAG_DENSE))) return APEXW_ERR_ARG;
    if (kind == 1 && (t->flags & APEXW_FLAG_ULTRA)) return APEXW_ERR_ARG;
    if (kind == 2 && !apexw_q8_fast_eligible(t->flags, t->block)) return APEXW_ERR_DTYPE;
    if (!(t->flags & APEXW_FLAG_DENSE) && !t->m_scale) return APEXW_ERR_ARG;
    if (!(t->flags & (APEXW_FLAG_DENSE | APEXW_FLAG_ULTRA)) && !t->v_scale) return APEXW_ERR_ARG;
  } else {
    return APEXW_ERR_ARG;
  }
  if (!(t->flags & APEXW_FLAG_SCALAR)) {
    const uintptr_t a = (uintptr_t)t->p | (uintptr_t)t->g | (uintptr_t)t->m | (uintptr_t)t->v;
    if (a & 15u) return APEXW_ERR_ALIGN;
  }
  return APEXW_OK;
}

// The scalar checks of one step launch (kind: APEXW_LAUNCH_COMPACT / _Q8 / _ULTRA /
// _FACTORED), shared by the step entry points and apexw_check_launch.
static int launch_args_status(int32_t kind, int32_t n_tensors, int64_t n_units, int64_t n_fast_units,
                              int64_t n_fast_f32_units, const apexw_hparams* hp) {
  if (n_tensors <= 0 || n_units < 0 || !hp_ok(hp)) return APEXW_ERR_ARG;
  switch (kind) {
    case APEXW_LAUNCH_COMPACT:
      if (n_fast_units || n_fast_f32_units) return APEXW_ERR_ARG;
      // cautious: the counts of apexw_compact_cautious_count, in the cold and replayed orders
      if ((hp->flags & APEXW_HP_CAUTIOUS) && (hp->mode == APEXW_MODE_NATIVE || ((uintptr_t)hp->counts & 7u)))
        return APEXW_ERR_ARG;
      // nesterov: the cold and replayed orders, with the host's step scalars in gain_hi / gain_lo
      if ((hp->flags & APEXW_HP_NESTEROV) &&
          (hp->mode == APEXW_MODE_NATIVE || hp->mode == APEXW_MODE_SINGLE || (hp->flags & APEXW_HP_AMP)))
        return APEXW_ERR_ARG;
      // lion: the cold and replayed orders, alone (it takes the place of the AdamW update)
      if ((hp->flags & APEXW_HP_LION) &&
          (hp->mode == APEXW_MODE_NATIVE || hp->mode == APEXW_MODE_SINGLE ||
           (hp->flags & (APEXW_HP_NESTEROV | APEXW_HP_CAUTIOUS | APEXW_HP_AMSGRAD | APEXW_HP_SLOW))))
        return APEXW_ERR_ARG;
      // beta3: the cold and replayed orders with the host's slow_ratio (no device AMP), not with cautious
      if ((hp->flags & APEXW_HP_SLOW) &&
          (hp->mode == APEXW_MODE_NATIVE || (hp->flags & (APEXW_HP_CAUTIOUS | APEXW_HP_AMP))))
        return APEXW_ERR_ARG;
      // grads of another dtype than their parameters: the cold and replayed orders (torch._fused_adamw_
      // refuses them, and so does the native mode)
      if ((hp->flags & APEXW_HP_GRAD_DTYPES) && (hp->mode == APEXW_MODE_NATIVE || hp->mode == APEXW_MODE_SINGLE))
        return APEXW_ERR_ARG;
      return APEXW_OK;
    case APEXW_LAUNCH_ULTRA:
      if (n_fast_units || n_fast_f32_units ||
          (hp->flags & (APEXW_HP_AMSGRAD | APEXW_HP_LION | APEXW_HP_SLOW | APEXW_HP_GRAD_DTYPES)))
        return APEXW_ERR_ARG;
      return (hp->mode == APEXW_MODE_NATIVE || hp->mode == APEXW_MODE_SINGLE) ? APEXW_ERR_ARG : APEXW_OK;
    case APEXW_LAUNCH_Q8:
      if (n_fast_units < 0 || n_fast_f32_units < 0 || n_fast_units + n_fast_f32_units > n_units) return APEXW_ERR_ARG;
      if (hp->mode == APEXW_MODE_NATIVE ||
          (hp->flags & (APEXW_HP_AMSGRAD | APEXW_HP_LION | APEXW_HP_SLOW | APEXW_HP_GRAD_DTYPES)))
        return APEXW_ERR_ARG;
      if (hp->mode == APEXW_MODE_SINGLE && (n_fast_units || n_fast_f32_units)) return APEXW_ERR_ARG;
      return APEXW_OK;
    case APEXW_LAUNCH_CAUTIOUS:
      if (n_fast_units || n_fast_f32_units) return APEXW_ERR_ARG;
      if (!(hp->flags & APEXW_HP_CAUTIOUS) || !hp->counts) return APEXW_ERR_ARG;
      if (hp->mode == APEXW_MODE_NATIVE || hp->mode == APEXW_MODE_SINGLE) return APEXW_ERR_ARG;
      return ((uintptr_t)hp->counts & 7u) ? APEXW_ERR_ALIGN : APEXW_OK;
    case APEXW_LAUNCH_FACTORED:
      if (n_fast_units || n_fast_f32_units ||
          (hp->flags & (APEXW_HP_AMSGRAD | APEXW_HP_LION | APEXW_HP_SLOW | APEXW_HP_GRAD_DTYPES)))
        return APEXW_ERR_ARG;
      if (hp->mode == APEXW_MODE_SINGLE || hp->mode == APEXW_MODE_NATIVE) return APEXW_ERR_ARG;
      return (hp->flags & APEXW_HP_AMP) ? APEXW_ERR_ARG : APEXW_OK;   // factored steps take host-read AMP scalars
    default:
      return APEXW_ERR_ARG;
  }
}

int apexw_check_launch(int32_t kind, int32_t n_tensors, int64_t n_units, int64_t n_fast_units,
                       int64_t n_fast_f32_units, const apexw_hparams* hp) {
  return launch_args_status(kind, n_tensors, n_units, n_fast_units, n_fast_f32_units, hp);
}

int apexw_compact_step(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units, int64_t n_units,
                       const apexw_hparams* hp, void* stream) {
  if (!tensors || !units) return APEXW_ERR_ARG;
  const int st = launch_args_status(APEXW_LAUNCH_COMPACT, n_tensors, n_units, 0, 0, hp);
  if (st != APEXW_OK || n_units == 0) return st;
  return apexw_launch_compact(tensors, n_units, units, hp, (hipStream_t)stream);
}

int apexw_q8_cautious_count(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units, int64_t n_units,
                            const apexw_hparams* hp, void* stream) {
  if (!tensors || !units) return APEXW_ERR_ARG;
  const int st = launch_args_status(APEXW_LAUNCH_CAUTIOUS, n_tensors, n_units, 0, 0, hp);
  if (st != APEXW_OK) return st;
  return apexw_launch_q8_cautious_count(tensors, n_tensors, units, n_units, hp, (hipStream_t)stream);
}

int apexw_compact_cautious_count(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units,
                                 int64_t n_units, const apexw_hparams* hp, void* stream) {
  if (!tensors || !units) return APEXW_ERR_ARG;
  const int st = launch_args_status(APEXW_LAUNCH_CAUTIOUS, n_tensors, n_units, 0, 0, hp);
  if (st != APEXW_OK) return st;
  return apexw_launch_compact_cautious_count(tensors, n_tensors, units, n_units, hp, (hipStream_t)stream);
}

int apexw_ultra_step(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units, int64_t n_units,
                     const apexw_hparams* hp, void* stream) {
  if (!tensors || !units) return APEXW_ERR_ARG;
  const int st = launch_args_status(APEXW_LAUNCH_ULTRA, n_tensors, n_units, 0, 0, hp);
  if (st != APEXW_OK || n_units == 0) return st;
  return apexw_launch_ultra(tensors, n_units, units, hp, (hipStream_t)stream);
}

int apexw_q8_step(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units, int64_t n_units,
                  int64_t n_fast_units, int64_t n_fast_f32_units, const apexw_hparams* hp, void* stream) {
  if (!tensors || !units) return APEXW_ERR_ARG;
  int st = launch_args_status(APEXW_LAUNCH_Q8, n_tensors, n_units, n_fast_units, n_fast_f32_units, hp);
  if (st != APEXW_OK) return st;
  if (n_fast_units > 0)
    st = apexw_launch_q8_fast(tensors, n_fast_units, units, hp, APEXW_BF16, (hipStream_t)stream);
  if (st == APEXW_OK && n_fast_f32_units > 0)
    st = apexw_launch_q8_fast(tensors, n_fast_f32_units, units + n_fast_units, hp, APEXW_F32, (hipStream_t)stream);
  const int64_t done = n_fast_units + n_fast_f32_units, rest = n_units - done;
  if (st == APEXW_OK && rest > 0)
    st = apexw_launch_q8(tensors, rest, units + done, hp, (hipStream_t)stream);
  return st;
}

int64_t apexw_factored_layout(apexw_fv_tensor* fv, int32_t n_fv, int64_t* n_bands, int64_t* n_col_blocks) {
  if (!fv || n_fv <= 0 || !n_bands || !n_col_blocks) return -APEXW_ERR_ARG;
  int64_t ws = 0, bands = 0, cbs = 0;
  for (int32_t i = 0; i < n_fv; ++i) {
    apexw_fv_tensor& e = fv[i];
    if (e.rows <= 0 || e.cols <= 0 || (e.flags & ~APEXW_FV_SUM_COLS)) return -APEXW_ERR_ARG;
    if (i > 0 && e.tensor <= fv[i - 1].tensor) return -APEXW_ERR_ARG;
    const int64_t nb = (e.rows + APEXW_FV_BAND_ROWS - 1) / APEXW_FV_BAND_ROWS;
    e.ws = ws;
    e.band0 = (int32_t)bands;
    e.cb0 = (int32_t)cbs;
    // band sums + inverse row mean, per-band column partials, column square roots; each 16-byte aligned
    auto r4 = [](int64_t x) { return (x + 3) & ~(int64_t)3; };
    ws += r4(nb + 1) + r4(nb * e.cols) + r4(e.cols);
    bands += nb;
    cbs += ((int64_t)e.cols + 63) / 64;   // finalisation column blocks of 64
    if (bands > INT32_MAX || cbs > INT32_MAX) return -APEXW_ERR_ARG;
  }
  *n_bands = bands;
  *n_col_blocks = cbs;
  return ws;
}

int apexw_factored_step(const apexw_tensor* tensors, int32_t n_tensors, const apexw_fv_tensor* fv, int32_t n_fv,
                        int64_t n_bands, int64_t n_col_blocks, const apexw_unit* units, int64_t n_units,
                        const int64_t* range_ends, float* workspace, const apexw_hparams* hp, void* stream) {
  if (!tensors || !fv || !workspace || n_fv <= 0 || n_fv > n_tensors) return APEXW_ERR_ARG;
  if (launch_args_status(APEXW_LAUNCH_FACTORED, n_tensors, n_units, 0, 0, hp) != APEXW_OK) return APEXW_ERR_ARG;
  if (n_bands < n_fv || n_bands > INT32_MAX || n_col_blocks < n_fv || n_col_blocks + n_fv > INT32_MAX) return APEXW_ERR_ARG;
  if (n_units < 0 || (n_units > 0 && !units) || !range_ends) return APEXW_ERR_ARG;
  int64_t prev = 0;
  for (int r = 0; r < APEXW_FV_UNIT_RANGES; ++r) {
    if (range_ends[r] < prev || range_ends[r] > n_units) return APEXW_ERR_ARG;
    prev = range_ends[r];
  }
  if (prev != n_units) return APEXW_ERR_ARG;
  return apexw_launch_factored(tensors, fv, n_fv, n_bands, n_col_blocks, units, range_ends, workspace, hp,
                               (hipStream_t)stream);
}

int apexw_gemm_nt_bf16(const void* a, const void* b, const void* et, void* c, void* ct, int32_t m, int32_t n,
                       int32_t k, int32_t lda, int32_t ldb, int32_t lde, int32_t ldc, int32_t ldct, int32_t batch,
                       int64_t stride_a, int64_t stride_b, int64_t stride_e, int64_t stride_c, int64_t stride_ct,
                       float alpha, float beta, void* stream) {
  if (!a || !b || (!c && !ct) || (beta != 0.0f && !et)) return APEXW_ERR_ARG;
  if (m <= 0 || n <= 0 || k <= 0 || batch <= 0 || batch > 65535) return APEXW_ERR_ARG;
  if (m % APEXW_GEMM_TILE || n % APEXW_GEMM_TILE || k % APEXW_GEMM_KTILE) return APEXW_ERR_ARG;
  // operand rows must cover the tile extents they are read over
  if (lda < k || ldb < k || (c && ldc < n) || (ct && ldct < m) || (et && lde < m)) return APEXW_ERR_ARG;
  if (lda > APEXW_GEMM_MAX_LD || ldb > APEXW_GEMM_MAX_LD || (et && lde > APEXW_GEMM_MAX_LD) ||
      (c && ldc > APEXW_GEMM_MAX_LD) || (ct && ldct > APEXW_GEMM_MAX_LD))
    return APEXW_ERR_ARG;
  if ((lda | ldb | (et ? lde : 0) | (c ? ldc : 0) | (ct ? ldct : 0)) & 7) return APEXW_ERR_ALIGN;
  const uintptr_t al = (uintptr_t)a | (uintptr_t)b | (uintptr_t)et | (uintptr_t)c | (uintptr_t)ct;
  if (al & 15u) return APEXW_ERR_ALIGN;
  if ((stride_a | stride_b | stride_e | stride_c | stride_ct) & 7) return APEXW_ERR_ALIGN;
  return apexw_launch_gemm_nt((const uint16_t*)a, (const uint16_t*)b, (const uint16_t*)et, (uint16_t*)c,
                              (uint16_t*)ct, m, n, k, lda, ldb, lde, ldc, ldct, batch, stride_a, stride_b, stride_e,
                              stride_c, stride_ct, alpha, beta, (hipStream_t)stream);
}

namespace {

constexpr int kTile = APEXW_GEMM_TILE;

// Epilogue kind of one problem, or minus a status when it is invalid.
int gemm_problem_kind(const apexw_gemm_problem& p) {
  const bool sym = p.flags & APEXW_GEMM_SYM, kn = p.flags & APEXW_GEMM_B_KN, add_b = p.flags & APEXW_GEMM_ADD_B;
  const bool apply = p.flags & APEXW_GEMM_APPLY;
  const bool add = p.beta != 0.0f;
  if (!p.a || !p.b || (!p.c && !p.ct && !apply)) return -APEXW_ERR_ARG;
  constexpr uint32_t kKnown = APEXW_GEMM_SYM | APEXW_GEMM_B_KN | APEXW_GEMM_ADD_B | APEXW_GEMM_APPLY |
                              APEXW_GEMM_APPLY_T | APEXW_GEMM_APPLY_WD | APEXW_GEMM_PANEL;
  if ((p.flags & ~kKnown) || p.reserved || p.reserved2) return -APEXW_ERR_ARG;
  if (apply) {
    // the X' product only (X as [K x N] rows, or X^T as the [N x K] operand, which may
    // also write O^T); p covered by O
    if (!add_b || (kn && p.ct) || !p.p) return -APEXW_ERR_ARG;
    if (p.p_dtype != APEXW_F32 && p.p_dtype != APEXW_BF16 && p.p_dtype != APEXW_F16) return -APEXW_ERR_DTYPE;
    const bool t = p.flags & APEXW_GEMM_APPLY_T;
    if (p.p_rows <= 0 || p.p_cols <= 0 || (t ? (p.p_cols > p.m || p.p_rows > p.n) : (p.p_rows > p.m || p.p_cols > p.n)))
      return -APEXW_ERR_ARG;
    if (((uintptr_t)p.p) & (p.p_dtype == APEXW_F32 ? 3u : 1u)) return -APEXW_ERR_ALIGN;
  } else if (p.p || p.p_dtype || p.p_rows || p.p_cols || p.wd_factor != 0.0f || p.neg_lr != 0.0f ||
             (p.flags & (APEXW_GEMM_APPLY_T | APEXW_GEMM_APPLY_WD))) {
    return -APEXW_ERR_ARG;
  }
  if (add_b ? (p.et || !add || p.alpha != 1.0f || p.m > p.k) : (add && !p.et)) return -APEXW_ERR_ARG;
  if (kn && (sym || p.ct)) return -APEXW_ERR_ARG;
  if (p.m <= 0 || p.n <= 0 || p.k <= 0) return -APEXW_ERR_ARG;
  if (p.m % kTile || p.n % kTile || p.k % APEXW_GEMM_KTILE) return -APEXW_ERR_ARG;
  if (p.m / kTile > 2048 || p.n / kTile > 2048) return -APEXW_ERR_ARG;
  const bool read_e = add && !add_b;
  if (p.lda < p.k || p.ldb < (kn ? p.n : p.k) || (p.c && p.ldc < p.n) || (p.ct && p.ldct < p.m) ||
      (read_e && p.lde < p.m))
    return -APEXW_ERR_ARG;
  const int32_t lds[5] = {p.lda, p.ldb, read_e ? p.lde : 0, p.c ? p.ldc : 0, p.ct ? p.ldct : 0};
  const int32_t ld_align = (p.flags & APEXW_GEMM_PANEL) ? 31 : 7;
  for (int32_t ld : lds) {
    if (ld > APEXW_GEMM_MAX_LD) return -APEXW_ERR_ARG;
    if (ld & ld_align) return -APEXW_ERR_ALIGN;
  }
  const uintptr_t al = (uintptr_t)p.a | (uintptr_t)p.b | (uintptr_t)(read_e ? p.et : nullptr) | (uintptr_t)p.c |
                       (uintptr_t)p.ct;
  if (al & 15u) return -APEXW_ERR_ALIGN;
  if (sym) {
    if (p.m != p.n || p.a != p.b || p.lda != p.ldb || !p.c || p.ct != p.c || p.ldct != p.ldc) return -APEXW_ERR_ARG;
  }
  // the applied update goes through the row-major epilogue (writing c too when given)
  return (p.c || apply ? APEXW_GEMM_OUT_C : 0) | (p.ct ? APEXW_GEMM_OUT_CT : 0) | (add ? APEXW_GEMM_ADD : 0) |
         (kn ? APEXW_GEMM_KIND_NN : 0) | ((p.flags & APEXW_GEMM_PANEL) ? APEXW_GEMM_KIND_PANEL : 0);
}

int64_t gemm_problem_tiles(const apexw_gemm_problem& p) {
  const int64_t tm = p.m / kTile, tn = p.n / kTile;
  return (p.flags & APEXW_GEMM_SYM) ? tm * (tm + 1) / 2 : tm * tn;
}

}  // namespace

int64_t apexw_gemm_grouped_items(const apexw_gemm_problem* problems, int32_t n_problems) {
  if (!problems || n_problems <= 0 || n_problems > 256) return -APEXW_ERR_ARG;
  int64_t n = 0;
  for (int32_t i = 0; i < n_problems; ++i) {
    const int kind = gemm_problem_kind(problems[i]);
    if (kind < 0) return kind;
    n += gemm_problem_tiles(problems[i]);
  }
  return n;
}

namespace {

// Makespan of one XCD's queue under the dispatcher's list scheduling: items
// start in order, each on the CU that frees first.
int64_t queue_makespan(const std::vector<int64_t>& costs, int cus) {
  std::priority_queue<int64_t, std::vector<int64_t>, std::greater<int64_t>> free_at;
  for (int c = 0; c < cus; ++c) free_at.push(0);
  int64_t end = 0;
  for (int64_t c : costs) {
    const int64_t t = free_at.top() + c;
    free_at.pop();
    free_at.push(t);
    end = std::max(end, t);
  }
  return end;
}

}  // namespace

int apexw_gemm_grouped_schedule(const apexw_gemm_problem* problems, int32_t n_problems, uint32_t* items,
                                int64_t n_items, int32_t cus_per_queue, int64_t* n_items_out,
                                int32_t* queue_offsets, int32_t* n_workgroups, int32_t* kind) {
  if (!items || !queue_offsets || !n_workgroups || !kind || !n_items_out) return APEXW_ERR_ARG;
  if (cus_per_queue < 0 || cus_per_queue > 1024) return APEXW_ERR_ARG;
  const int64_t want = apexw_gemm_grouped_items(problems, n_problems);
  if (want < 0) return (int)-want;
  if (n_items < 2 * want || want >= INT32_MAX / 2) return APEXW_ERR_ARG;
  const int kind0 = gemm_problem_kind(problems[0]);
  for (int32_t i = 1; i < n_problems; ++i)
    if (gemm_problem_kind(problems[i]) != kind0) return APEXW_ERR_ARG;

  // Per problem, the tiles in locality order (bands of 4 tile rows, each band
  // column by column, so a run of consecutive tiles shares A row panels and B
  // column panels) are cut into one contiguous band per queue: all XCDs work on
  // the same matrix at once and share its panels in the Infinity Cache.  A
  // problem's T tiles give every queue T / 8 of them, and the T % 8 left over go
  // to the next queues in rotation across problems, so queues stay within about
  // one tile of each other.  Inside a queue the longest tiles come first: the
  // XCD starts them first and fills in with the short ones.
  //
  // Cost model, in twentieths of a K tile: a whole tile costs its K tiles plus
  // 2 per epilogue stream (C, Ct, E); a 128-row half costs 0.55 of the K part
  // (half the MFMAs, the same number of pipelined K steps) and half the
  // epilogue.  With cus_per_queue > 0 (the CUs of one XCD), each queue's last
  // s tiles are split into halves for the s that minimises the simulated
  // makespan (ties keep fewer halves): 400 equal tiles on 32 CUs take 12.5
  // rounds instead of 13 once the last 16 are halved.
  struct Item {
    uint32_t code;
    int64_t cost, half_cost;
  };
  constexpr int nq = APEXW_GEMM_QUEUES;
  const int64_t epi = 2 * (((kind0 & APEXW_GEMM_OUT_C) != 0) + ((kind0 & APEXW_GEMM_OUT_CT) != 0) +
                           ((kind0 & APEXW_GEMM_ADD) != 0));
  std::vector<std::vector<Item>> band(nq);
  std::vector<Item> tiles;
  int rotate = 0;
  for (int32_t pi = 0; pi < n_problems; ++pi) {
    const apexw_gemm_problem& p = problems[pi];
    const int tiles_m = p.m / kTile, tiles_n = p.n / kTile;
    const bool sym = (p.flags & APEXW_GEMM_SYM) != 0;
    const int64_t kt = p.k / APEXW_GEMM_KTILE;
    const int64_t cost = 20 * (kt + epi), half_cost = 11 * kt + 10 * epi;
    tiles.clear();
    for (int g0 = 0; g0 < tiles_m; g0 += 4)
      for (int tn = 0; tn < tiles_n; ++tn)
        for (int tm = g0; tm < std::min(g0 + 4, tiles_m); ++tm) {
          if (sym && tm > tn) continue;
          tiles.push_back({((uint32_t)pi << 24) | ((uint32_t)tm << 11) | (uint32_t)tn, cost, half_cost});
        }
    const size_t t = tiles.size(), base = t / nq, rem = t % nq;
    size_t off = 0;
    for (int q = 0; q < nq; ++q) {
      const size_t take = base + (((size_t)((q - rotate + nq) % nq)) < rem ? 1 : 0);
      band[q].insert(band[q].end(), tiles.begin() + off, tiles.begin() + off + take);
      off += take;
    }
    rotate = (int)((rotate + rem) % nq);
  }
  int64_t pos = 0;
  size_t longest = 0;
  std::vector<int64_t> costs;
  for (int x = 0; x < nq; ++x) {
    std::vector<Item>& b = band[x];
    std::stable_sort(b.begin(), b.end(), [](const Item& l, const Item& r) { return l.cost > r.cost; });
    size_t split = 0;
    if (cus_per_queue > 0) {
      int64_t best = -1;
      const size_t most = std::min(b.size(), (size_t)cus_per_queue);
      for (size_t s = 0; s <= most; ++s) {
        costs.clear();
        for (size_t i = 0; i + s < b.size(); ++i) costs.push_back(b[i].cost);
        for (size_t i = b.size() - s; i < b.size(); ++i) {
          costs.push_back(b[i].half_cost);
          costs.push_back(b[i].half_cost);
        }
        const int64_t span = queue_makespan(costs, cus_per_queue);
        if (best < 0 || span < best) {
          best = span;
          split = s;
        }
      }
    }
    queue_offsets[x] = (int32_t)pos;
    for (size_t i = 0; i + split < b.size(); ++i) items[pos++] = b[i].code;
    for (size_t i = b.size() - split; i < b.size(); ++i) {
      items[pos++] = b[i].code | (1u << 22);
      items[pos++] = b[i].code | (2u << 22);
    }
    longest = std::max(longest, (size_t)(pos - queue_offsets[x]));
  }
  queue_offsets[nq] = (int32_t)pos;
  if ((int64_t)longest * nq > INT32_MAX) return APEXW_ERR_ARG;
  *n_items_out = pos;
  *n_workgroups = (int32_t)(longest * nq);
  *kind = kind0;
  return APEXW_OK;
}

int apexw_gemm_nt_grouped(const apexw_gemm_problem* problems, const uint32_t* items, const int32_t* queue_offsets,
                          int32_t n_workgroups, int32_t kind, const apexw_amp_dyn* amp, void* stream) {
  if (!problems || !items || !queue_offsets) return APEXW_ERR_ARG;
  if ((uintptr_t)amp & 15u) return APEXW_ERR_ALIGN;
  if (n_workgroups <= 0 || n_workgroups % APEXW_GEMM_QUEUES) return APEXW_ERR_ARG;
  if (kind <= 0 || kind > 31 || !(kind & (APEXW_GEMM_OUT_C | APEXW_GEMM_OUT_CT))) return APEXW_ERR_ARG;
  if ((kind & APEXW_GEMM_KIND_NN) && (kind & APEXW_GEMM_OUT_CT)) return APEXW_ERR_ARG;
  if (((uintptr_t)problems | (uintptr_t)items | (uintptr_t)queue_offsets) & 3u) return APEXW_ERR_ALIGN;
  return apexw_launch_gemm_grouped(problems, items, queue_offsets, n_workgroups, kind, amp, (hipStream_t)stream);
}

int64_t apexw_muon_workspace_floats(int64_t rows, int64_t cols) {
  return rows > 0 && cols > 0 ? apexw_muon_partials(rows * cols) : 0;
}

int apexw_muon_prepare(float* buf, const void* g, int32_t g_dtype, int64_t rows, int64_t cols, float mu,
                       float one_minus_mu, int32_t nesterov, float eps, float grad_inv_scale, void* x, void* xt,
                       int64_t ldx, int64_t ldxt, int32_t layout, float* workspace, const apexw_amp_dyn* amp,
                       void* stream) {
  if (!buf || !g || !x || !workspace || rows <= 0 || cols <= 0) return APEXW_ERR_ARG;
  if ((uintptr_t)amp & 15u) return APEXW_ERR_ALIGN;
  if (g_dtype != APEXW_F32 && g_dtype != APEXW_BF16 && g_dtype != APEXW_F16) return APEXW_ERR_DTYPE;
  if (layout != APEXW_LAYOUT_ROWS && layout != APEXW_LAYOUT_PANEL) return APEXW_ERR_ARG;
  // work matrix X is [min x max], X^T is [max x min] (optional)
  const int64_t lo = rows < cols ? rows : cols, hi = rows < cols ? cols : rows;
  if (ldx < hi || (xt && ldxt < lo)) return APEXW_ERR_ARG;
  if (layout == APEXW_LAYOUT_PANEL && ((ldx & 31) || (xt && (ldxt & 31)))) return APEXW_ERR_ALIGN;
  if (!amp && !(grad_inv_scale > 0.0f)) return APEXW_ERR_ARG;
  return apexw_launch_muon_prepare(buf, g, g_dtype, rows, cols, mu, one_minus_mu, nesterov, eps, grad_inv_scale,
                                   (uint16_t*)x, (uint16_t*)xt, ldx, ldxt, layout == APEXW_LAYOUT_PANEL, workspace,
                                   amp, (hipStream_t)stream);
}

int apexw_muon_apply(void* p, int32_t p_dtype, const void* u, int64_t rows, int64_t cols, int64_t ldu,
                     int32_t layout, int32_t u_transposed, float wd_factor, int32_t apply_wd, float neg_lr_eff,
                     const apexw_amp_dyn* amp, void* stream) {
  if ((uintptr_t)amp & 15u) return APEXW_ERR_ALIGN;
  if (!p || !u || rows <= 0 || cols <= 0 || ldu < (u_transposed ? rows : cols)) return APEXW_ERR_ARG;
  if (layout != APEXW_LAYOUT_ROWS && layout != APEXW_LAYOUT_PANEL) return APEXW_ERR_ARG;
  if (layout == APEXW_LAYOUT_PANEL && (ldu & 31)) return APEXW_ERR_ALIGN;
  if ((rows + 63) / 64 > 65535) return APEXW_ERR_ARG;   // grid y of the transposing kernel
  if (p_dtype != APEXW_F32 && p_dtype != APEXW_BF16 && p_dtype != APEXW_F16) return APEXW_ERR_DTYPE;
  return apexw_launch_muon_apply(p, p_dtype, (const uint16_t*)u, rows, cols, ldu, layout == APEXW_LAYOUT_PANEL,
                                 u_transposed != 0, wd_factor, apply_wd, neg_lr_eff, amp, (hipStream_t)stream);
}

int apexw_muon_coordwise(float* buf, const void* g, int32_t g_dtype, void* p, int32_t p_dtype, int64_t n, float mu,
                         float one_minus_mu, int32_t nesterov, float grad_inv_scale, float wd_factor,
                         int32_t apply_wd, float neg_lr, const apexw_amp_dyn* amp, void* stream) {
  if (!buf || !g || !p || n <= 0) return APEXW_ERR_ARG;
  if ((uintptr_t)amp & 15u) return APEXW_ERR_ALIGN;
  if (g_dtype != APEXW_F32 && g_dtype != APEXW_BF16 && g_dtype != APEXW_F16) return APEXW_ERR_DTYPE;
  if (p_dtype != APEXW_F32 && p_dtype != APEXW_BF16 && p_dtype != APEXW_F16) return APEXW_ERR_DTYPE;
  if (!amp && !(grad_inv_scale > 0.0f)) return APEXW_ERR_ARG;
  return apexw_launch_muon_coordwise(buf, g, g_dtype, p, p_dtype, n, mu, one_minus_mu, nesterov, grad_inv_scale,
                                     wd_factor, apply_wd, neg_lr, amp, (hipStream_t)stream);
}

int apexw_grad_clip_coef(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units, int64_t n_units,
                         int64_t unit_size, const int64_t* unit_begin, float* unit_partial, float* tensor_norm,
                         float clip, float grad_inv_scale, uint32_t flags, float* coef, const apexw_amp_dyn* amp,
                         const apexw_row_means* rows, void* stream) {
  if (!tensors || !units || !unit_begin || !unit_partial || !tensor_norm || !coef) return APEXW_ERR_ARG;
  if (n_tensors <= 0 || n_units < 0 || unit_size < 0 || !(clip > 0.0f)) return APEXW_ERR_ARG;
  if ((flags & APEXW_HP_UNSCALE) && !amp && !apexw_inv_scale_ok(grad_inv_scale)) return APEXW_ERR_ARG;
  return apexw_launch_clip(tensors, n_tensors, units, n_units, unit_size, unit_begin, unit_partial, tensor_norm, clip,
                           grad_inv_scale, flags, coef, amp, rows, (hipStream_t)stream);
}

int apexw_check_grad_prep(const apexw_grad_prep* d) {
  if (!d || !d->g || !d->out || d->n <= 0 || d->row_len < 0 || d->reserved) return APEXW_ERR_ARG;
  if (d->dtype != APEXW_F32 && d->dtype != APEXW_BF16 && d->dtype != APEXW_F16) return APEXW_ERR_DTYPE;
  if (d->row_len > 0 && d->n % d->row_len) return APEXW_ERR_ARG;
  const int64_t size = d->dtype == APEXW_F32 ? 4 : 2;
  const uintptr_t g = (uintptr_t)d->g, o = (uintptr_t)d->out;
  if (g < o + (uintptr_t)(d->n * size) && o < g + (uintptr_t)(d->n * size)) return APEXW_ERR_ARG;   // aliasing
  if ((g | o) & (uintptr_t)(size - 1)) return APEXW_ERR_ALIGN;
  return APEXW_OK;
}

int apexw_check_row_means(const apexw_grad_prep* d) {
  if (!d || !d->g || !d->out || d->n <= 0 || d->row_len <= 0 || d->reserved) return APEXW_ERR_ARG;
  if (d->dtype != APEXW_F32 && d->dtype != APEXW_BF16 && d->dtype != APEXW_F16) return APEXW_ERR_DTYPE;
  if (d->n % d->row_len) return APEXW_ERR_ARG;
  const int64_t size = d->dtype == APEXW_F32 ? 4 : 2;
  const uintptr_t g = (uintptr_t)d->g, o = (uintptr_t)d->out;
  const uintptr_t g_end = g + (uintptr_t)(d->n * size), o_end = o + (uintptr_t)(d->n / d->row_len * 4);
  if (g < o_end && o < g_end) return APEXW_ERR_ARG;   // the means must not alias the grad
  if ((g & (uintptr_t)(size - 1)) || (o & 3u)) return APEXW_ERR_ALIGN;
  return APEXW_OK;
}

int64_t apexw_grad_prep_units(const apexw_grad_prep* d) {
  const int st = apexw_check_grad_prep(d);
  if (st != APEXW_OK) return -st;
  return d->row_len > 0 ? d->n / d->row_len : (d->n + APEXW_GRAD_PREP_CHUNK - 1) / APEXW_GRAD_PREP_CHUNK;
}

int apexw_grad_prepare(const apexw_grad_prep* preps, int32_t n_preps, const apexw_unit* units, int64_t n_units,
                       float grad_inv_scale, uint32_t flags, const apexw_amp_dyn* amp, void* stream) {
  if (!preps || !units || n_preps <= 0 || n_units < 0) return APEXW_ERR_ARG;
  if (flags & ~(APEXW_HP_SANITIZE | APEXW_HP_UNSCALE)) return APEXW_ERR_ARG;
  if ((flags & APEXW_HP_UNSCALE) && !amp && !apexw_inv_scale_ok(grad_inv_scale)) return APEXW_ERR_ARG;
  return apexw_launch_grad_prep(preps, units, n_units, grad_inv_scale, flags, amp, (hipStream_t)stream);
}

int apexw_grad_row_means(const apexw_grad_prep* preps, int32_t n_preps, const apexw_unit* units, int64_t n_units,
                         float grad_inv_scale, uint32_t flags, const apexw_amp_dyn* amp, void* stream) {
  if (!preps || !units || n_preps <= 0 || n_units < 0) return APEXW_ERR_ARG;
  if (flags & ~(APEXW_HP_SANITIZE | APEXW_HP_UNSCALE)) return APEXW_ERR_ARG;
  if ((flags & APEXW_HP_UNSCALE) && !amp && !apexw_inv_scale_ok(grad_inv_scale)) return APEXW_ERR_ARG;
  return apexw_launch_row_means(preps, units, n_units, grad_inv_scale, flags, amp, (hipStream_t)stream);
}

int apexw_amp_prepare(const float* found_inf, const float* grad_scale, int32_t* skips, int32_t skips_folded,
                      const apexw_amp_launch* launches, int32_t n_launches, apexw_amp_dyn* dyn, void* stream) {
  if (!found_inf || !grad_scale || !skips || !launches || !dyn) return APEXW_ERR_ARG;
  if (n_launches <= 0 || n_launches > APEXW_AMP_MAX_LAUNCHES || skips_folded < 0) return APEXW_ERR_ARG;
  for (int i = 0; i < n_launches; ++i) {
    const apexw_amp_launch& l = launches[i];
    if (l.kind > 1 || l.reserved || !(l.step >= 1.0) || !(l.beta1 >= 0.0 && l.beta1 < 1.0) ||
        !(l.beta2 >= 0.0 && l.beta2 < 1.0))
      return APEXW_ERR_ARG;
  }
  if (((uintptr_t)found_inf | (uintptr_t)grad_scale | (uintptr_t)skips) & 3u) return APEXW_ERR_ALIGN;
  if ((uintptr_t)dyn & 15u) return APEXW_ERR_ALIGN;
  return apexw_launch_amp_prepare(found_inf, grad_scale, skips, skips_folded, launches, n_launches, dyn,
                                  (hipStream_t)stream);
}

}  // extern "C"
