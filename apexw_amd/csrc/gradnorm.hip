// Global-L2 gradient clip coefficient on the device (gfx950).
//
// Restates the clip of _prepare_grads (apexw/optimizer.py:242-256) without the
// host synchronisation: per-tensor norms (torch._foreach_norm rounds each norm
// to the grad dtype), the L2 norm of those norms, and
// coef = min(clip / (total + 1e-6), 1).  The step kernels read the coefficient
// from device memory and scale the grads in registers.
//
// Three short launches, deterministic (no atomics):
//   1. one wavefront per work unit of the chunk table -> sum of squares
//   2. one wavefront per tensor sums its (contiguous) units -> rounded norm
//   3. one workgroup combines the tensor norms -> coefficient
#include <mutex>

#include "common.h"

namespace {

// squares of sanitize(g) (when san), unscaled in the grad dtype when unscale
// (AMP grads are unscaled before the clip, apexw/optimizer.py:227-237).
// Sanitizing changes only NaN / +-Inf grads, and one of those makes the lane's sum
// non-finite: the sum is formed without it, and a lane whose sum is not finite
// (rare) forms it again with it.
template <int GD, int N>
APEXW_DEV float sumsq_vals(const float (&g)[N], bool san, bool unscale, float inv, float acc, bool gc,
                           const float (&mean)[N]) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
    float x = san ? sanitize<GD>(g[j]) : g[j];
    if (unscale) x = rnd<GD>(x * inv);
    if (gc) x = rnd<GD>(x - mean[j]);
    acc = fmaf(x, x, acc);
  }
  return acc;
}

// Row means (APEXW_FLAG_GC: `means` holds one per row of rl elements) of the 8
// elements from e0; zeros for a tensor that is not centralized (means == nullptr).
APEXW_DEV void clip_means8(const apexw_tensor& t, const float* means, int64_t rl, int64_t e0, float (&mean)[8]) {
  if (!means) {
#pragma unroll
    for (int j = 0; j < 8; ++j) mean[j] = 0.0f;
    return;
  }
  const int64_t rows = t.n / rl;
  if (rl >= 8) {
    // at most one row boundary inside the 8 elements
    const int64_t row = e0 / rl, col = e0 - row * rl;
    const float m0 = means[row < rows ? row : rows - 1];
    const float m1 = (col + 8 > rl && row + 1 < rows) ? means[row + 1] : m0;
#pragma unroll
    for (int j = 0; j < 8; ++j) mean[j] = col + j < rl ? m0 : m1;
    return;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t r = (e0 + j) / rl;
    mean[j] = means[r < rows ? r : rows - 1];
  }
}

// means / rl: the tensor's row means and row length when it is centralized, else
// nullptr / 0
template <int GD>
APEXW_DEV float unit_sumsq(const apexw_tensor& t, int64_t start, int64_t cnt, bool san, bool unscale, float inv,
                           const float* means, int64_t rl) {
  const int lane = lane_id();
  const bool vec = !(t.flags & APEXW_FLAG_SCALAR) && (start % 8) == 0;
  float acc = 0.0f;
  const bool gc = means != nullptr;
  if (vec && cnt == 2048 && !gc) {
    // a whole 2048-element unit: the wave's four 8-element loads per lane are issued
    // together (centralized tensors take the loop below, in the same summation order,
    // so that their row means do not hold registers here)
    float g[4][8];
    const float none[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 4; ++k) load8<GD>(t.g, start + k * 512 + lane * 8, g[k]);
#pragma unroll
    for (int k = 0; k < 4; ++k) acc = sumsq_vals<GD, 8>(g[k], false, unscale, inv, acc, false, none);
    if (san && !(acc - acc == 0.0f)) {
      // rare: a NaN / Inf grad in this lane's elements; read them again (the values need
      // not stay in registers past the first pass) and form the sum with them sanitized
      acc = 0.0f;
      for (int k = 0; k < 4; ++k) {
        float h[8];
        load8<GD>(t.g, start + k * 512 + lane * 8, h);
        acc = sumsq_vals<GD, 8>(h, true, unscale, inv, acc, false, none);
      }
    }
    return wave_sum(acc);
  }
  for (int pass = 0; pass < 2; ++pass) {
    const bool s = pass == 1;
    acc = 0.0f;
    for (int64_t rel = (int64_t)lane * 8; rel < cnt; rel += 64 * 8) {
      const int64_t e0 = start + rel;
      const int c = (cnt - rel) < 8 ? (int)(cnt - rel) : 8;
      float g[8];
      if (vec && c == 8) {
        load8<GD>(t.g, e0, g);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) g[j] = j < c ? load1<GD>(t.g, e0 + j) : 0.0f;
      }
      float mean[8];
      clip_means8(t, means, rl, e0, mean);
      acc = sumsq_vals<GD, 8>(g, s, unscale, inv, acc, gc, mean);
    }
    if (!san || acc - acc == 0.0f) break;
  }
  return wave_sum(acc);
}

__global__ __launch_bounds__(256) void sumsq_kernel(const apexw_tensor* __restrict__ tensors,
                                                    const apexw_unit* __restrict__ units, int64_t n_units,
                                                    int64_t unit_size, float* __restrict__ partial, uint32_t flags,
                                                    float inv, const apexw_amp_dyn* __restrict__ amp,
                                                    const apexw_row_means* __restrict__ rows) {
  if (amp) inv = amp->grad_inv_scale;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const bool san = flags & APEXW_HP_SANITIZE, unscale = flags & APEXW_HP_UNSCALE;
  // a workgroup walks a contiguous chunk of 64 units, its waves interleaved, one
  // workgroup per chunk (the dispatcher balances the tail): at C4 (2.08 B grads)
  // 0.631 ms against 0.679 ms for a resident grid striding by 4 units
  for (int64_t base = (int64_t)blockIdx.x * 64; base < n_units; base += (int64_t)gridDim.x * 64)
  for (int64_t u = base + wave, u_end = base + 64 < n_units ? base + 64 : n_units; u < u_end; u += 4) {
    const apexw_unit un = units[u];
    const apexw_tensor& t = tensors[un.tensor];
    const int64_t us = unit_size > 0 ? unit_size : (t.block > 0 ? (int64_t)t.block : 64);
    const int64_t start = (int64_t)un.unit * us;
    const int64_t cnt = (t.n - start) < us ? (t.n - start) : us;
    const uint32_t gd = (t.flags >> APEXW_FLAG_GDT_SHIFT) & 3u;
    // a centralized tensor's row means: its descriptor's own fields (compact tables) or
    // its entry of the side table (8-bit / ultra tables)
    const float* means = nullptr;
    int64_t rl = 0;
    if (t.flags & APEXW_FLAG_GC) {
      means = rows ? rows[un.tensor].means : t.m_scale;
      rl = rows ? rows[un.tensor].row_len : (int64_t)t.block;
    }
    float s;
    if (gd == APEXW_F32) s = unit_sumsq<APEXW_F32>(t, start, cnt, san, unscale, inv, means, rl);
    else if (gd == APEXW_BF16) s = unit_sumsq<APEXW_BF16>(t, start, cnt, san, unscale, inv, means, rl);
    else s = unit_sumsq<APEXW_F16>(t, start, cnt, san, unscale, inv, means, rl);
    if (lane_id() == 0) partial[u] = s;
  }
}

__global__ __launch_bounds__(256) void tensor_norm_kernel(const apexw_tensor* __restrict__ tensors, int32_t n_tensors,
                                                          const int64_t* __restrict__ unit_begin,
                                                          const float* __restrict__ partial, float* __restrict__ norm) {
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const int64_t stride = (int64_t)gridDim.x * 4;
  for (int64_t t = (int64_t)blockIdx.x * 4 + wave; t < n_tensors; t += stride) {
    float acc = 0.0f;
    for (int64_t u = unit_begin[t] + lane_id(); u < unit_begin[t + 1]; u += 64) acc += partial[u];
    acc = wave_sum(acc);
    const uint32_t gd = (tensors[t].flags >> APEXW_FLAG_GDT_SHIFT) & 3u;
    float nrm = sqrtf(acc);
    nrm = gd == APEXW_BF16 ? rnd<APEXW_BF16>(nrm) : (gd == APEXW_F16 ? rnd<APEXW_F16>(nrm) : nrm);
    if (lane_id() == 0) norm[t] = nrm;
  }
}

__global__ __launch_bounds__(1024) void clip_coef_kernel(const float* __restrict__ norm, int32_t n_tensors, float clip,
                                                         float* __restrict__ coef) {
  __shared__ float s_part[16];
  float acc = 0.0f;
  for (int32_t t = threadIdx.x; t < n_tensors; t += blockDim.x) acc = fmaf(norm[t], norm[t], acc);
  acc = wave_sum(acc);
  if (lane_id() == 0) s_part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float tot = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) tot += s_part[w];
    const float total = sqrtf(tot);
    float c = clip / (total + 1e-6f);
    // torch.clamp(c, max=1) then "multiply only if c < 1": NaN / >= 1 leave grads unscaled
    coef[0] = (c < 1.0f) ? c : 1.0f;
  }
}

// ---------------------------------------------------------------------------
// Gradient preparation (sanitize, AMP unscale, centralization), one 256-thread
// workgroup per unit: a row of a centralized grad (sum pass, then subtract and
// store; the row is re-read from L2) or a 2048-element chunk of any other grad.
// ---------------------------------------------------------------------------
template <int GD> APEXW_DEV float prep_value(const void* g, int64_t i, bool san, bool unscale, float inv) {
  float x = load1<GD>(g, i);
  if (san) x = sanitize<GD>(x);
  if (unscale) x = rnd<GD>(x * inv);
  return x;
}

template <int GD> APEXW_DEV void prep_vec8(const void* g, int64_t i, bool san, bool unscale, float inv,
                                           float (&x)[8]) {
  load8<GD>(g, i, x);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (san) x[j] = sanitize<GD>(x[j]);
    if (unscale) x[j] = rnd<GD>(x[j] * inv);
  }
}

// Elements [lo, hi) of a grad: the 8-aligned middle [a, b) in 8-element vectors
// (16-byte bf16 / 32-byte fp32 accesses) when both buffers are aligned for
// them, the ragged ends element by element.
struct PrepSpan {
  int64_t a, b;
};
template <int GD> APEXW_DEV PrepSpan prep_span(const apexw_grad_prep& d, int64_t lo, int64_t hi) {
  constexpr uintptr_t align = GD == APEXW_F32 ? 31 : 15;
  if ((((uintptr_t)d.g | (uintptr_t)d.out) & align) != 0) return {hi, hi};
  const int64_t a = (lo + 7) & ~(int64_t)7, b = hi & ~(int64_t)7;
  return a < b ? PrepSpan{a, b} : PrepSpan{hi, hi};
}

template <int GD>
APEXW_DEV void prep_unit(const apexw_grad_prep& d, int64_t unit, bool san, bool unscale, float inv, float* red) {
  const int tid = threadIdx.x;
  const bool row = d.row_len > 0;
  const int64_t lo = row ? unit * d.row_len : unit * APEXW_GRAD_PREP_CHUNK;
  const int64_t hi = row ? lo + d.row_len : (lo + APEXW_GRAD_PREP_CHUNK < d.n ? lo + APEXW_GRAD_PREP_CHUNK : d.n);
  const PrepSpan sp = prep_span<GD>(d, lo, hi);
  // ragged ends: [lo, a) and [b, hi) (the whole range when not vectorized)
  const int64_t head = sp.a - lo, n_end = head + (hi - sp.b);
  float mean = 0.0f;
  if (row) {
    float s = 0.0f;
    for (int64_t i = sp.a + (int64_t)tid * 8; i < sp.b; i += 2048) {
      float x[8];
      prep_vec8<GD>(d.g, i, san, unscale, inv, x);
#pragma unroll
      for (int j = 0; j < 8; ++j) s += x[j];
    }
    for (int64_t k = tid; k < n_end; k += 256) {
      const int64_t i = k < head ? lo + k : sp.b + (k - head);
      s += prep_value<GD>(d.g, i, san, unscale, inv);
    }
    s = wave_sum(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    // torch's mean: sum in fp32, divided by the count, result in the grad dtype
    mean = rnd<GD>(((red[0] + red[1]) + (red[2] + red[3])) / (float)d.row_len);
  }
  // second pass (the row is re-read from L2): subtract the mean and store
  for (int64_t i = sp.a + (int64_t)tid * 8; i < sp.b; i += 2048) {
    float x[8];
    prep_vec8<GD>(d.g, i, san, unscale, inv, x);
    if (row) {
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = rnd<GD>(x[j] - mean);
    }
    store8<GD>(d.out, i, x);
  }
  for (int64_t k = tid; k < n_end; k += 256) {
    const int64_t i = k < head ? lo + k : sp.b + (k - head);
    const float x = prep_value<GD>(d.g, i, san, unscale, inv);
    store1<GD>(d.out, i, row ? rnd<GD>(x - mean) : x);
  }
}

// Row means only (the fold of centralization into the step kernels): one wave per
// row of a descriptor with row_len > 0; d.out is a float array of one mean per
// row, each the grad dtype's rounding of the fp32 row sum over row_len of the
// sanitized, unscaled grads.  A lane sums its 8-element vectors (four loads issued
// before they are added; eight measured slower at C3), then the wave's lanes are
// summed.
template <int GD>
APEXW_DEV void mean_row(const apexw_grad_prep& d, int64_t row, bool san, bool unscale, float inv) {
  const int lane = lane_id();
  const int64_t lo = row * d.row_len, hi = lo + d.row_len;
  const PrepSpan sp = prep_span<GD>(d, lo, hi);
  const int64_t head = sp.a - lo, n_end = head + (hi - sp.b);
  float s = 0.0f;
  int64_t i = sp.a + (int64_t)lane * 8;
  for (; i + 3 * 512 < sp.b; i += 4 * 512) {
    float x[4][8];
#pragma unroll
    for (int q = 0; q < 4; ++q) prep_vec8<GD>(d.g, i + q * 512, san, unscale, inv, x[q]);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int j = 0; j < 8; ++j) s += x[q][j];
  }
  for (; i < sp.b; i += 512) {
    float x[8];
    prep_vec8<GD>(d.g, i, san, unscale, inv, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) s += x[j];
  }
  for (int64_t k = lane; k < n_end; k += 64) {
    const int64_t i = k < head ? lo + k : sp.b + (k - head);
    s += prep_value<GD>(d.g, i, san, unscale, inv);
  }
  s = wave_sum(s);
  if (lane == 0) ((float*)d.out)[row] = rnd<GD>(s / (float)d.row_len);
}

__global__ __launch_bounds__(256) void row_means_kernel(const apexw_grad_prep* __restrict__ preps,
                                                        const apexw_unit* __restrict__ units, int64_t n_units,
                                                        float inv, uint32_t flags,
                                                        const apexw_amp_dyn* __restrict__ amp) {
  if (amp) inv = amp->grad_inv_scale;
  const bool san = flags & APEXW_HP_SANITIZE, unscale = flags & APEXW_HP_UNSCALE;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  // workgroup b takes a contiguous chunk of 64 rows, its waves interleaved
  for (int64_t base = (int64_t)blockIdx.x * 64; base < n_units; base += (int64_t)gridDim.x * 64)
  for (int64_t u = base + wave, u_end = base + 64 < n_units ? base + 64 : n_units; u < u_end; u += 4) {
    const apexw_unit un = units[u];
    const apexw_grad_prep& d = preps[un.tensor];
    if (d.dtype == APEXW_F32) mean_row<APEXW_F32>(d, un.unit, san, unscale, inv);
    else if (d.dtype == APEXW_BF16) mean_row<APEXW_BF16>(d, un.unit, san, unscale, inv);
    else mean_row<APEXW_F16>(d, un.unit, san, unscale, inv);
  }
}

__global__ __launch_bounds__(256) void grad_prep_kernel(const apexw_grad_prep* __restrict__ preps,
                                                        const apexw_unit* __restrict__ units, int64_t n_units,
                                                        float inv, uint32_t flags,
                                                        const apexw_amp_dyn* __restrict__ amp) {
  __shared__ float red[4];
  if (amp) inv = amp->grad_inv_scale;
  const bool san = flags & APEXW_HP_SANITIZE, unscale = flags & APEXW_HP_UNSCALE;
  for (int64_t u = blockIdx.x; u < n_units; u += gridDim.x) {
    const apexw_unit un = units[u];
    const apexw_grad_prep& d = preps[un.tensor];
    if (d.dtype == APEXW_F32) prep_unit<APEXW_F32>(d, un.unit, san, unscale, inv, red);
    else if (d.dtype == APEXW_BF16) prep_unit<APEXW_BF16>(d, un.unit, san, unscale, inv, red);
    else prep_unit<APEXW_F16>(d, un.unit, san, unscale, inv, red);
    __syncthreads();   // red is reused by the next unit
  }
}

}  // namespace

int apexw_launch_grad_prep(const apexw_grad_prep* preps, const apexw_unit* units, int64_t n_units, float inv,
                           uint32_t flags, const apexw_amp_dyn* amp, hipStream_t stream) {
  if (n_units <= 0) return APEXW_OK;
  const int64_t want = n_units < 65536 ? n_units : 65536;
  hipLaunchKernelGGL(grad_prep_kernel, dim3((unsigned)want), dim3(256), 0, stream, preps, units, n_units, inv, flags,
                     amp);
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

int apexw_launch_clip(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units, int64_t n_units,
                      int64_t unit_size, const int64_t* unit_begin, float* unit_partial, float* tensor_norm,
                      float clip, float inv, uint32_t flags, float* coef, const apexw_amp_dyn* amp,
                      const apexw_row_means* rows, hipStream_t stream);

int apexw_launch_row_means(const apexw_grad_prep* preps, const apexw_unit* units, int64_t n_units, float inv,
                           uint32_t flags, const apexw_amp_dyn* amp, hipStream_t stream) {
  if (n_units <= 0) return APEXW_OK;
  const int64_t chunks = (n_units + 63) / 64;
  const unsigned grid = (unsigned)(chunks < INT32_MAX ? chunks : INT32_MAX);
  hipLaunchKernelGGL(row_means_kernel, dim3(grid), dim3(256), 0, stream, preps, units, n_units, inv, flags, amp);
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

// ---------------------------------------------------------------------------
// Allocation-free clip coefficient: the per-unit partials and per-tensor norms
// live in this file-scope device array instead of caller workspace.  Each GPU
// holds its own copy; its device address is looked up once per device with
// hipGetSymbolAddress (the array's name is only a host-side stand-in).
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[APEXW_NOALLOC_CLIP_MAX_UNITS + APEXW_NOALLOC_CLIP_MAX_TENSORS];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kScratchDevices];

// Device address of `scratch` on device dev, or nullptr if it cannot be had.  A
// lookup that fails is not cached: the next call tries again.
float* scratch_on_device(int dev) {
  if (dev < 0 || dev >= kScratchDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev]) return g_scratch_ptr[dev];
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return nullptr;
  // hipGetSymbolAddress answers for the calling thread's current device
  if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
  void* ptr = nullptr;
  const bool ok = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) == hipSuccess && ptr;
  if (cur != dev) (void)hipSetDevice(cur);
  if (ok) g_scratch_ptr[dev] = (float*)ptr;
  return ok ? (float*)ptr : nullptr;
}

}  // namespace

extern "C" int apexw_grad_clip_coef_noalloc(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units,
                                            int64_t n_units, int64_t unit_size, const int64_t* unit_begin,
                                            float clip, float grad_inv_scale, uint32_t flags, float* coef,
                                            const apexw_amp_dyn* amp, void* stream) {
  if (!tensors || !units || !unit_begin || !coef) return APEXW_ERR_ARG;
  if (n_tensors <= 0 || n_units < 0 || unit_size < 0 || !(clip > 0.0f)) return APEXW_ERR_ARG;
  if ((flags & APEXW_HP_UNSCALE) && !amp && !apexw_inv_scale_ok(grad_inv_scale)) return APEXW_ERR_ARG;
  if (n_units > APEXW_NOALLOC_CLIP_MAX_UNITS || n_tensors > APEXW_NOALLOC_CLIP_MAX_TENSORS) return APEXW_ERR_SIZE;
  // the array of the GPU the kernels run on: the stream's device (the null stream is
  // the current device's)
  int dev = -1;
  if (stream) {
    if (hipStreamGetDevice((hipStream_t)stream, &dev) != hipSuccess) return APEXW_ERR_ARG;
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return APEXW_ERR_LAUNCH;
  }
  float* ptr = scratch_on_device(dev);
  if (!ptr) return APEXW_ERR_LAUNCH;
  return apexw_launch_clip(tensors, n_tensors, units, n_units, unit_size, unit_begin, ptr,
                           ptr + APEXW_NOALLOC_CLIP_MAX_UNITS, clip, grad_inv_scale, flags, coef, amp, nullptr,
                           (hipStream_t)stream);
}

int apexw_launch_clip(const apexw_tensor* tensors, int32_t n_tensors, const apexw_unit* units, int64_t n_units,
                      int64_t unit_size, const int64_t* unit_begin, float* unit_partial, float* tensor_norm,
                      float clip, float inv, uint32_t flags, float* coef, const apexw_amp_dyn* amp,
                      const apexw_row_means* rows, hipStream_t stream) {
  if (n_units > 0) {
    const int64_t chunks = (n_units + 63) / 64;
    const int grid_units = (int)(chunks < INT32_MAX ? chunks : INT32_MAX);
    hipLaunchKernelGGL(sumsq_kernel, dim3(grid_units), dim3(256), 0, stream, tensors, units, n_units, unit_size,
                       unit_partial, flags, inv, amp, rows);
  }
  if (n_tensors > 0) {
    const int grid_tensors = apexw_resident_grid((const void*)tensor_norm_kernel, n_tensors);
    hipLaunchKernelGGL(tensor_norm_kernel, dim3(grid_tensors), dim3(256), 0, stream, tensors, n_tensors, unit_begin,
                       unit_partial, tensor_norm);
  }
  hipLaunchKernelGGL(clip_coef_kernel, dim3(1), dim3(1024), 0, stream, tensor_norm, n_tensors, clip, coef);
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

// ---------------------------------------------------------------------------
// GradScaler's scale and found_inf read on the device (apexw_amp_prepare): one
// thread turns them and the host's step counts into each launch's scalars.
// ---------------------------------------------------------------------------
namespace {

struct AmpLaunches {
  apexw_amp_launch l[APEXW_AMP_MAX_LAUNCHES];
};

__global__ __launch_bounds__(64) void amp_prepare_kernel(const float* __restrict__ found_inf,
                                                         const float* __restrict__ grad_scale,
                                                         int32_t* __restrict__ skips, int32_t folded, AmpLaunches ls,
                                                         int32_t n, apexw_amp_dyn* __restrict__ dyn) {
  if (threadIdx.x != 0) return;
  const uint32_t skip = *found_inf != 0.0f ? 1u : 0u;
  const int32_t s = *skips;
  if (skip) *skips = s + 1;
  const float inv = 1.0f / *grad_scale;
  for (int i = 0; i < n; ++i) {
    const apexw_amp_launch& L = ls.l[i];
    const double t = L.step - (double)(s - folded);
    const double bc1 = 1.0 - pow(L.beta1, t), bc2 = 1.0 - pow(L.beta2, t);
    const double bc2s = sqrt(bc2);
    apexw_amp_dyn d;
    if (L.kind == 1) {
      d.step_size = (float)(L.lr / bc1);
      d.eps_scaled = (float)L.eps;
      d.bc2_sqrt = (float)bc2s;
    } else {
      d.step_size = (float)(L.lr * bc2s / bc1);
      d.eps_scaled = (float)(L.eps * bc2s);
      d.bc2_sqrt = (float)bc2s;
    }
    d.grad_inv_scale = inv;
    d.skip = skip;
    d.reserved[0] = d.reserved[1] = d.reserved[2] = 0u;
    dyn[i] = d;
  }
}

}  // namespace

int apexw_launch_amp_prepare(const float* found_inf, const float* grad_scale, int32_t* skips, int32_t folded,
                             const apexw_amp_launch* launches, int32_t n, apexw_amp_dyn* dyn, hipStream_t stream) {
  AmpLaunches ls;
  for (int i = 0; i < n; ++i) ls.l[i] = launches[i];
  hipLaunchKernelGGL(amp_prepare_kernel, dim3(1), dim3(64), 0, stream, found_inf, grad_scale, skips, folded, ls, n,
                     dyn);
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}
