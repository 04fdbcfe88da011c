// Bandwidth probes for bench.py --ceiling (libapexw_probe.so; not part of the
// optimizer's C ABI).  They measure what HBM delivers on this GPU for the
// streams the optimizer step moves, with no arithmetic in the way:
//   * copy / read-only / write-only of one buffer, each wave moving chunk_kib
//     KiB contiguous per iteration (16-byte nontemporal accesses);
//   * the 8-bit step's exact access pattern (bf16 p and g, NF4 m, quad log-u8
//     v, two fp32 scales per 2048-element block; p, m, v and the scales written
//     back), blocks_per_wave consecutive blocks per wave per iteration, with
//     the stored values changed (an xor) so that no store can be dropped;
//   * the compact step's pattern (bf16 p, g, m and a dense or quad bf16 v read,
//     p, m and v written back): one 512-element group per wave and work item,
//     8 consecutive elements per lane, the work items of a workgroup's waves
//     consecutive, as the compact step kernel walks its units.
#include <hip/hip_runtime.h>
#include <stdint.h>

#define PROBE_API extern "C" __attribute__((visibility("default")))

namespace {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
#define GPTR(T, p) ((__attribute__((address_space(1))) T*)(p))

template <typename T> __device__ __forceinline__ T nt_load(const void* a) {
  return __builtin_nontemporal_load(GPTR(const T, a));
}
template <typename T> __device__ __forceinline__ void nt_store(void* a, T x) {
  __builtin_nontemporal_store(x, GPTR(T, a));
}

// U = 16-byte vectors per lane per iteration (a wave moves U KiB contiguous)
template <int U> __global__ __launch_bounds__(256) void copy_kernel(const u32x4* a, u32x4* b, int64_t n) {
  const int lane = threadIdx.x & 63;
  const int64_t chunks = n / (64 * U);
  for (int64_t c = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); c < chunks; c += (int64_t)gridDim.x * 4) {
    u32x4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = nt_load<u32x4>(a + c * 64 * U + u * 64 + lane);
#pragma unroll
    for (int u = 0; u < U; ++u) nt_store<u32x4>(b + c * 64 * U + u * 64 + lane, x[u]);
  }
}

template <int U> __global__ __launch_bounds__(256) void read_kernel(const u32x4* a, uint32_t* sink, int64_t n) {
  const int lane = threadIdx.x & 63;
  const int64_t chunks = n / (64 * U);
  uint32_t acc = 0;
  for (int64_t c = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); c < chunks; c += (int64_t)gridDim.x * 4) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const u32x4 x = nt_load<u32x4>(a + c * 64 * U + u * 64 + lane);
      acc ^= x.x ^ x.y ^ x.z ^ x.w;
    }
  }
  if (acc == 0x5eed5eedu) sink[0] = acc;   // keeps the loads; practically never stores
}

template <int U> __global__ __launch_bounds__(256) void write_kernel(u32x4* b, int64_t n) {
  const int lane = threadIdx.x & 63;
  const int64_t chunks = n / (64 * U);
  for (int64_t c = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); c < chunks; c += (int64_t)gridDim.x * 4) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const u32x4 x = {(uint32_t)c, (uint32_t)u, (uint32_t)lane, 1u};
      nt_store<u32x4>(b + c * 64 * U + u * 64 + lane, x);
    }
  }
}

// The 8-bit step's streams per 2048-element block, lane layout of the step kernel
// (8 consecutive elements per lane in each of four 512-element slices).
template <int BPW>
__global__ __launch_bounds__(256) void q8_pattern_kernel(uint16_t* p, const uint16_t* g, uint8_t* m, uint8_t* v,
                                                         float* ms, float* vs, int64_t nblk) {
  const int lane = threadIdx.x & 63;
  for (int64_t b0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * BPW; b0 + BPW <= nblk;
       b0 += (int64_t)gridDim.x * 4 * BPW) {
    u32x4 pw[BPW][4], gw[BPW][4];
    uint32_t mw[BPW][4], vw[BPW][2];
    float sa[BPW], sc[BPW];
#pragma unroll
    for (int q = 0; q < BPW; ++q) {
      const int64_t s = (b0 + q) * 2048;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t e = s + k * 512 + lane * 8;
        pw[q][k] = nt_load<u32x4>(p + e);
        gw[q][k] = nt_load<u32x4>(g + e);
        mw[q][k] = nt_load<uint32_t>(m + (e >> 1));
      }
      vw[q][0] = nt_load<uint16_t>(v + ((s + lane * 8) >> 2)) | (nt_load<uint16_t>(v + ((s + 512 + lane * 8) >> 2)) << 16);
      vw[q][1] = nt_load<uint16_t>(v + ((s + 1024 + lane * 8) >> 2)) |
                 (nt_load<uint16_t>(v + ((s + 1536 + lane * 8) >> 2)) << 16);
      sa[q] = GPTR(const float, ms)[b0 + q];
      sc[q] = GPTR(const float, vs)[b0 + q];
    }
#pragma unroll
    for (int q = 0; q < BPW; ++q) {
      const int64_t s = (b0 + q) * 2048;
      uint32_t acc = 0;
      u32x4 o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        o[k] = pw[q][k] ^ gw[q][k] ^ 0x00010001u;
        acc ^= mw[q][k] ^ o[k].x;
      }
      acc ^= vw[q][0] ^ vw[q][1];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t e = s + k * 512 + lane * 8;
        nt_store(p + e, o[k]);
        nt_store(m + (e >> 1), mw[q][k] ^ o[k].y ^ 1u);
        nt_store(v + (e >> 2), (uint16_t)((k & 1 ? vw[q][k >> 1] >> 16 : vw[q][k >> 1]) ^ o[k].z ^ 1u));
      }
      if (lane == 0) {
        GPTR(float, ms)[b0 + q] = sa[q] + (float)(acc & 1u) + 1.0f;
        GPTR(float, vs)[b0 + q] = sc[q] + 1.0f;
      }
    }
  }
}

template <bool QUAD>
__global__ __launch_bounds__(256) void compact_pattern_kernel(uint16_t* p, const uint16_t* g, uint16_t* m, uint16_t* v,
                                                              int64_t n_items) {
  const int lane = threadIdx.x & 63;
  for (int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); w < n_items; w += (int64_t)gridDim.x * 4) {
    const int64_t e = w * 512 + lane * 8;
    const u32x4 a = nt_load<u32x4>(p + e), b = nt_load<u32x4>(g + e), c = nt_load<u32x4>(m + e);
    if constexpr (QUAD) {
      const uint32_t d = nt_load<uint32_t>(v + (e >> 2));
      nt_store(p + e, a ^ b ^ 1u);
      nt_store(m + e, c ^ b ^ 2u);
      nt_store(v + (e >> 2), d ^ b.x ^ 3u);
    } else {
      const u32x4 d = nt_load<u32x4>(v + e);
      nt_store(p + e, a ^ b ^ 1u);
      nt_store(m + e, c ^ b ^ 2u);
      nt_store(v + e, d ^ b ^ 3u);
    }
  }
}

bool ok(int grid) { return grid > 0 && grid <= (1 << 20); }

}  // namespace

// bytes: a multiple of 16 * 64 * chunk_kib; chunk_kib in {1, 4, 16}.  Returns 0 when launched.
PROBE_API int apexw_probe_copy(const void* src, void* dst, int64_t bytes, int32_t chunk_kib, int32_t grid, void* stream) {
  if (!src || !dst || bytes <= 0 || !ok(grid)) return 1;
  const int64_t n = bytes / 16;
  hipStream_t s = (hipStream_t)stream;
  if (chunk_kib == 1) hipLaunchKernelGGL(copy_kernel<1>, dim3(grid), dim3(256), 0, s, (const u32x4*)src, (u32x4*)dst, n);
  else if (chunk_kib == 4) hipLaunchKernelGGL(copy_kernel<4>, dim3(grid), dim3(256), 0, s, (const u32x4*)src, (u32x4*)dst, n);
  else if (chunk_kib == 16) hipLaunchKernelGGL(copy_kernel<16>, dim3(grid), dim3(256), 0, s, (const u32x4*)src, (u32x4*)dst, n);
  else return 1;
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

PROBE_API int apexw_probe_read(const void* src, int64_t bytes, int32_t chunk_kib, int32_t grid, uint32_t* sink,
                               void* stream) {
  if (!src || !sink || bytes <= 0 || !ok(grid)) return 1;
  const int64_t n = bytes / 16;
  hipStream_t s = (hipStream_t)stream;
  if (chunk_kib == 4) hipLaunchKernelGGL(read_kernel<4>, dim3(grid), dim3(256), 0, s, (const u32x4*)src, sink, n);
  else if (chunk_kib == 16) hipLaunchKernelGGL(read_kernel<16>, dim3(grid), dim3(256), 0, s, (const u32x4*)src, sink, n);
  else return 1;
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

PROBE_API int apexw_probe_write(void* dst, int64_t bytes, int32_t chunk_kib, int32_t grid, void* stream) {
  if (!dst || bytes <= 0 || !ok(grid)) return 1;
  const int64_t n = bytes / 16;
  hipStream_t s = (hipStream_t)stream;
  if (chunk_kib == 4) hipLaunchKernelGGL(write_kernel<4>, dim3(grid), dim3(256), 0, s, (u32x4*)dst, n);
  else if (chunk_kib == 16) hipLaunchKernelGGL(write_kernel<16>, dim3(grid), dim3(256), 0, s, (u32x4*)dst, n);
  else return 1;
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

// p, g: n_blocks * 2048 bf16; m: n_blocks * 1024 bytes; v: n_blocks * 512 bytes; ms, vs: n_blocks floats.
// blocks_per_wave in {1, 4}; only whole groups of blocks_per_wave blocks are touched.
PROBE_API int apexw_probe_q8_pattern(void* p, const void* g, void* m, void* v, float* ms, float* vs, int64_t n_blocks,
                                     int32_t blocks_per_wave, int32_t grid, void* stream) {
  if (!p || !g || !m || !v || !ms || !vs || n_blocks <= 0 || !ok(grid)) return 1;
  hipStream_t s = (hipStream_t)stream;
  if (blocks_per_wave == 1)
    hipLaunchKernelGGL(q8_pattern_kernel<1>, dim3(grid), dim3(256), 0, s, (uint16_t*)p, (const uint16_t*)g,
                       (uint8_t*)m, (uint8_t*)v, ms, vs, n_blocks);
  else if (blocks_per_wave == 4)
    hipLaunchKernelGGL(q8_pattern_kernel<4>, dim3(grid), dim3(256), 0, s, (uint16_t*)p, (const uint16_t*)g,
                       (uint8_t*)m, (uint8_t*)v, ms, vs, n_blocks);
  else
    return 1;
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

// p, g, m: n_items * 512 bf16; v: the same (quad == 0) or n_items * 128 bf16 (quad == 1).
PROBE_API int apexw_probe_compact_pattern(void* p, const void* g, void* m, void* v, int64_t n_items, int32_t quad,
                                          int32_t grid, void* stream) {
  if (!p || !g || !m || !v || n_items <= 0 || !ok(grid) || (quad != 0 && quad != 1)) return 1;
  hipStream_t s = (hipStream_t)stream;
  if (quad)
    hipLaunchKernelGGL(compact_pattern_kernel<true>, dim3(grid), dim3(256), 0, s, (uint16_t*)p, (const uint16_t*)g,
                       (uint16_t*)m, (uint16_t*)v, n_items);
  else
    hipLaunchKernelGGL(compact_pattern_kernel<false>, dim3(grid), dim3(256), 0, s, (uint16_t*)p, (const uint16_t*)g,
                       (uint16_t*)m, (uint16_t*)v, n_items);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}
