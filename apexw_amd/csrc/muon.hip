// Muon on gfx950: fp32 momentum, Newton-Schulz with bf16 MFMA GEMMs, decoupled
// weight decay and the scaled orthogonalised update.
//
// Newton-Schulz (apexw/muon.py:102-108, :135-184), per iteration on the wide
// work matrix X [m x n], m <= n:
//   A  = X X^T                 (symmetric, K = n)
//   B  = c A A + b A           (symmetric, K = m)
//   X' = B X + a X             (K = m)
// Every product is computed as an "NT" GEMM (both operands K-contiguous): X is
// kept in both layouts, X [m x n] and X^T [n x m], so B X = B (X^T)^T reads X^T
// rows.  The epilogue of the last product writes X' in both layouts; the
// symmetric products are written through the transposed store (same matrix).
// Work matrices are zero-padded to multiples of the 256 x 256 tile; zero rows
// and columns stay zero through every product, so the kernel has no bounds
// checks.
#include "common.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) uint16_t u16x4;

constexpr int kBM = 256, kBN = 256, kBK = 64;
// LDS tiles are [rows x 64] bf16 with 128-byte rows; the eight 16-byte chunks of
// row r are stored XOR-swizzled (chunk c at slot c ^ (r & 7)), so the MFMA
// fragment reads of 8 consecutive rows hit 8 distinct bank groups.
APEXW_DEV int lds_off(int row, int chunk) { return row * kBK + ((chunk ^ (row & 7)) << 3); }

struct GemmArgs {
  const uint16_t* a;   // [M x K] row-major, ld lda
  const uint16_t* b;   // [N x K] row-major, ld ldb
  const uint16_t* et;  // addend, transposed: et[j * lde + i] is E[i][j] (may be null when beta == 0)
  uint16_t* c;         // [M x N] row-major output, ld ldc (may be null)
  uint16_t* ct;        // [N x M] transposed output, ld ldct (may be null)
  int64_t sa, sb, se, sc, sct;  // batch strides (elements)
  int32_t m, n, k, lda, ldb, lde, ldc, ldct;
  float alpha, beta;
};

APEXW_DEV float bf(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
APEXW_DEV uint16_t to_bf(float x) { return (uint16_t)f32_to_bf16_bits(x); }

typedef uint16_t LdsTile[kBM * kBK];

// global -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4): lane L's
// 16 bytes at gbase + voff land at LDS byte lds_base + 16 L.  Issued as inline
// assembly so that the compiler does not track it as an LDS write: it would
// otherwise make every later LDS read wait for it (it cannot tell the two
// stage buffers apart), serialising each K tile's prefetch with its math.  The
// kernel orders these copies itself: s_waitcnt vmcnt(0) and a barrier before a
// stage is read, and a stage is refilled only after the barrier that ends its
// last reads.
// M0 is written only here in these kernels (nothing else in them reads it); the
// clobber records that, and clang's note that it cannot preserve a reserved
// register across the statement does not apply.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
APEXW_DEV void lds_copy16(uint32_t lds_base, uint32_t voff, const void* gbase) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds_base), "v"(voff), "s"(gbase)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// A workgroup-uniform pointer held in SGPRs (the asm operand above needs one;
// a pointer loaded from a table is not known to be uniform by the compiler).
APEXW_DEV const uint16_t* uniform_ptr(const uint16_t* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const uint16_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

APEXW_DEV uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// One 256 x 256 output tile: O = alpha * A B^T + beta * E (bf16 in, fp32
// accumulate, bf16 out, round to nearest even).  A and B point at the tile's
// first row of each operand; Et, C and Ct at the tile's origin in their own
// layouts.  256 threads = 4 waves in a 2 x 2 arrangement, each owning a
// 128 x 128 block as 4 x 4 MFMA 32x32x16 accumulators; K tiles of 64 are
// double-buffered in LDS and loaded straight from global memory into LDS.
// Template flags select the epilogue: write O row-major (kC), transposed (kCt,
// skipped at run time when write_ct is false), add beta * E (kAdd).
template <bool kC, bool kCt, bool kAdd>
APEXW_DEV void gemm_tile(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, int32_t lda, int32_t ldb,
                         int32_t k, const uint16_t* __restrict__ Et, int32_t lde, uint16_t* __restrict__ C,
                         int32_t ldc, uint16_t* __restrict__ Ct, int32_t ldct, bool write_ct, float alpha,
                         float beta, LdsTile* s_a, LdsTile* s_b) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // global -> LDS without registers (global_load_lds_dwordx4): each wave
  // instruction fills 1 KB of LDS = 8 tile rows, lane L landing at byte 16 L.
  // Lane L of chunk q reads row 8 q + L / 8 at column chunk (L % 8) ^ (L / 8),
  // which is the swizzled slot L % 8 of that row.  Per K tile each wave issues
  // 8 instructions for A and 8 for B (chunks q = 8 wave + i).
  uint32_t goff_a[8], goff_b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 8 * (8 * wave + i) + (lane >> 3), chunk = (lane & 7) ^ (lane >> 3);
    goff_a[i] = (uint32_t)(row * lda + chunk * 8) * 2u;
    goff_b[i] = (uint32_t)(row * ldb + chunk * 8) * 2u;
  }
  // LDS byte address of this wave's first chunk in each stage (wave-uniform)
  const uint32_t lds_a0 = __builtin_amdgcn_readfirstlane(lds_address(&s_a[0][8 * wave * 512]));
  const uint32_t lds_b0 = __builtin_amdgcn_readfirstlane(lds_address(&s_b[0][8 * wave * 512]));
  constexpr uint32_t kStage = sizeof(LdsTile), kChunk = 512 * sizeof(uint16_t);
  const uint16_t* A_s = uniform_ptr(A);
  const uint16_t* B_s = uniform_ptr(B);
  auto issue_loads = [&](int buf, int k0) {
    const uint16_t* a0 = A_s + k0;
    const uint16_t* b0 = B_s + k0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      lds_copy16(lds_a0 + buf * kStage + i * kChunk, goff_a[i], a0);
      lds_copy16(lds_b0 + buf * kStage + i * kChunk, goff_b[i], b0);
    }
  };
  // the loads write LDS asynchronously: wait for this wave's, then the barrier
  // makes every wave's visible
  auto loads_done = [&]() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };

  f32x16 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f32x16{};

  // MFMA 32x32x16 operand layout: lane l supplies row (l % 32) and k = 8 (l / 32) .. +7.
  // Fragments are double-buffered in registers: the 8 LDS reads of k-step s + 1
  // are issued before the 16 MFMAs of step s.  sched_barrier(0) pins that order
  // (the scheduler would otherwise sink each read next to its first use and
  // expose the full LDS latency before every few MFMAs).
  const int frag_row = lane & 31, frag_c = lane >> 5;
  bf16x8 fa[2][4], fb[2][4];
  auto frags = [&](int buf, int s, int slot) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
      fa[slot][a] = *(const bf16x8*)&s_a[buf][lds_off(wm * 128 + a * 32 + frag_row, s * 2 + frag_c)];
#pragma unroll
    for (int b = 0; b < 4; ++b)
      fb[slot][b] = *(const bf16x8*)&s_b[buf][lds_off(wn * 128 + b * 32 + frag_row, s * 2 + frag_c)];
  };
  auto mma = [&](int slot) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[slot][a], fb[slot][b], acc[a][b], 0, 0, 0);
  };
#define APEXW_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

  const int k_tiles = k / kBK;
  issue_loads(0, 0);
  loads_done();
  __syncthreads();
  for (int kt = 0; kt < k_tiles; ++kt) {
    // stage buf ^ 1 was last read before the previous barrier: refill it with
    // tile kt + 1 while tile kt is multiplied
    const int buf = kt & 1;
    if (kt + 1 < k_tiles) issue_loads(buf ^ 1, (kt + 1) * kBK);
    frags(buf, 0, 0);
    APEXW_SCHED_FENCE();
    frags(buf, 1, 1);
    APEXW_SCHED_FENCE();
    mma(0);
    APEXW_SCHED_FENCE();
    frags(buf, 2, 0);
    APEXW_SCHED_FENCE();
    mma(1);
    APEXW_SCHED_FENCE();
    frags(buf, 3, 1);
    APEXW_SCHED_FENCE();
    mma(0);
    APEXW_SCHED_FENCE();
    mma(1);
    APEXW_SCHED_FENCE();
    loads_done();
    __syncthreads();
  }
#undef APEXW_SCHED_FENCE

  // Epilogue.  Accumulator register r of lane l holds row 8 (r / 4) + 4 (l / 32) + r % 4,
  // column l % 32 of its 32 x 32 block: four consecutive rows of one column per group.
  // After the last barrier the operand tiles are dead: each wave stages its
  // 128 x 128 block of O in its own 32 KB of LDS, then writes it row by row to C
  // and column by column to Ct, both as 16-byte stores along output rows.  The
  // stage keeps 16-byte chunks XOR-swizzled by row / 8 so that the row reads
  // (16 lanes per row) and the column reads (16 lanes down a column) each hit
  // distinct banks.  A wave reads back only what it wrote itself, and LDS keeps
  // one wave's accesses in order, so no barrier is needed.
  uint16_t* stage = (wave < 2 ? s_a[wave] : s_b[wave - 2]);
  auto swz = [](int r, int c) { return r * 128 + ((((c >> 3) ^ (r >> 3)) & 15) << 3) + (c & 7); };
  const int il0 = (lane >> 5) * 4, jl0 = lane & 31;           // within the wave's block
  const int gi0 = wm * 128 + il0, gj0 = wn * 128 + jl0;       // within the tile
#pragma unroll
  for (int a = 0; a < 4; ++a) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int jl = jl0 + b * 32;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int il = il0 + a * 32 + q * 8;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = alpha * acc[a][b][q * 4 + r];
        if constexpr (kAdd) {
          const u16x4 e = *APEXW_GLOBAL(const u16x4, Et + (uint32_t)((gj0 + b * 32) * lde + gi0 + a * 32 + q * 8));
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = fmaf(beta, bf(e[r]), v[r]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) stage[swz(il + r, jl)] = to_bf(v[r]);
      }
    }
  }
  if constexpr (kC) {
    uint16_t* __restrict__ Cw = C + (int64_t)(wm * 128) * ldc + wn * 128;
#pragma unroll 4
    for (int it = 0; it < 32; ++it) {
      const int c = it * 64 + lane, r = c >> 4, c16 = c & 15;
      const u32x4 v = *(const u32x4*)&stage[swz(r, c16 * 8)];
      __builtin_nontemporal_store(v, APEXW_GLOBAL(u32x4, Cw + (uint32_t)(r * ldc + c16 * 8)));
    }
  }
  if constexpr (kCt) {
    if (write_ct) {
      uint16_t* __restrict__ Ctw = Ct + (int64_t)(wn * 128) * ldct + wm * 128;
#pragma unroll 2
      for (int it = 0; it < 32; ++it) {
        // Ct row jl (= column jl of the block), elements il .. il + 7
        const int c = it * 64 + lane, jl = c >> 4, il = (c & 15) * 8;
        u32x4 v;
#pragma unroll
        for (int t = 0; t < 4; ++t)
          v[t] = (uint32_t)stage[swz(il + 2 * t, jl)] | ((uint32_t)stage[swz(il + 2 * t + 1, jl)] << 16);
        *APEXW_GLOBAL(u32x4, Ctw + (uint32_t)(jl * ldct + il)) = v;
      }
    }
  }
}

// Batched GEMM over one shape: one workgroup per output tile, blockIdx.y = batch entry.
template <bool kC, bool kCt, bool kAdd>
__global__ __launch_bounds__(256, 1) void gemm_nt_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) LdsTile s_a[2];
  __shared__ __attribute__((aligned(16))) LdsTile s_b[2];

  const int tiles_m = g.m / kBM, tiles_n = g.n / kBN, tiles = tiles_m * tiles_n;
  // Consecutive workgroups are dispatched round-robin over the 8 XCDs; give each
  // XCD a contiguous range of tiles, ordered in groups of 4 tile rows, so the A
  // and B panels a range touches stay in that XCD's L2.
  const int per_xcd = (tiles + 7) / 8;
  const int t = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  if (t >= tiles) return;
  constexpr int kGroup = 4;
  const int group = t / (kGroup * tiles_n), first_m = group * kGroup;
  const int gm = min(tiles_m - first_m, kGroup);
  const int in_group = t % (kGroup * tiles_n);
  const int tm = first_m + in_group % gm, tn = in_group / gm;

  const int64_t batch = blockIdx.y;
  const int64_t row0 = (int64_t)tm * kBM, col0 = (int64_t)tn * kBN;
  gemm_tile<kC, kCt, kAdd>(g.a + batch * g.sa + row0 * g.lda, g.b + batch * g.sb + col0 * g.ldb, g.lda, g.ldb, g.k,
                           kAdd ? g.et + batch * g.se + col0 * g.lde + row0 : nullptr, g.lde,
                           kC ? g.c + batch * g.sc + row0 * g.ldc + col0 : nullptr, g.ldc,
                           kCt ? g.ct + batch * g.sct + col0 * g.ldct + row0 : nullptr, g.ldct, true, g.alpha, g.beta,
                           s_a, s_b);
}

// Grouped GEMM: every problem of a launch (different shapes, K and operands)
// in one grid, one workgroup per output tile.  The tiles are split into
// kQueues queues, one per XCD: workgroups are dispatched round-robin over the
// 8 XCDs, so workgroup b runs on XCD b % 8 and computes tile b / 8 of queue
// b % 8.  Each XCD thus works through its own queue in order, a new workgroup
// starting on whichever of its CUs frees first; a queue is one contiguous band
// of tiles in locality order, longest first.  Workgroups past the end of their
// queue exit at once.  An item packs (problem << 24) | (tile row << 12) | tile
// column.  A symmetric problem (APEXW_GEMM_SYM) lists only tiles with
// row <= column and mirrors each off-diagonal tile through the transposed
// store (ct == c).
constexpr int kQueues = APEXW_GEMM_QUEUES;

template <bool kC, bool kCt, bool kAdd>
__global__ __launch_bounds__(256, 1) void gemm_nt_grouped_kernel(const apexw_gemm_problem* __restrict__ probs,
                                                                 const uint32_t* __restrict__ items,
                                                                 const int32_t* __restrict__ queue_offsets) {
  __shared__ __attribute__((aligned(16))) LdsTile s_a[2];
  __shared__ __attribute__((aligned(16))) LdsTile s_b[2];
  const int q = (int)(blockIdx.x % kQueues), i = (int)(blockIdx.x / kQueues);
  const int begin = queue_offsets[q];
  if (i >= queue_offsets[q + 1] - begin) return;
  const uint32_t code = items[begin + i];
  const apexw_gemm_problem& p = probs[code >> 24];
  const int tm = (int)((code >> 12) & 0xfffu), tn = (int)(code & 0xfffu);
  const int64_t row0 = (int64_t)tm * kBM, col0 = (int64_t)tn * kBN;
  const bool mirror = !(p.flags & APEXW_GEMM_SYM) || tm != tn;
  gemm_tile<kC, kCt, kAdd>((const uint16_t*)p.a + row0 * p.lda, (const uint16_t*)p.b + col0 * p.ldb, p.lda, p.ldb,
                           p.k, kAdd ? (const uint16_t*)p.et + col0 * p.lde + row0 : nullptr, p.lde,
                           kC ? (uint16_t*)p.c + row0 * p.ldc + col0 : nullptr, p.ldc,
                           kCt ? (uint16_t*)p.ct + col0 * p.ldct + row0 : nullptr, p.ldct, mirror, p.alpha, p.beta,
                           s_a, s_b);
}

// ---------------------------------------------------------------------------
// Momentum (apexw/muon.py:763-792, fp32 buffer): buf = buf * mu, then
// buf += (1 - mu) * g with g sanitized (NaN -> 0, +-Inf -> +-65504) and widened
// to fp32.  The NS input ("update source") is buf, or lerp(g, buf, mu) with
// Nesterov.  Per-block partial sums of squares of bf16(update source) give the
// Frobenius norm of the bf16 work matrix.
// ---------------------------------------------------------------------------
template <int GD> APEXW_DEV float muon_grad(const void* grad, int64_t i) {
  float g = load1<GD>(grad, i);
  if (__builtin_isnan(g)) return 0.0f;
  if (__builtin_isinf(g)) return g > 0.0f ? 65504.0f : -65504.0f;
  return g;
}

// torch.lerp(g, m, w): g + w (m - g) for w < 0.5, else m - (1 - w)(m - g), one fma each
APEXW_DEV float nesterov_source(float g, float m, float mu) {
  return mu < 0.5f ? fmaf(mu, m - g, g) : fmaf(mu - 1.0f, m - g, m);
}

// VEC: 8 elements per thread with 16-byte accesses (buf and grad 16-byte
// aligned); the n % 8 tail and unaligned tensors take the element-wise loop.
template <int GD, bool VEC>
__global__ __launch_bounds__(256) void muon_momentum_kernel(float* __restrict__ buf, const void* __restrict__ grad,
                                                            int64_t n, float mu, float one_minus_mu, int nesterov,
                                                            float* __restrict__ partial) {
  float s = 0.0f;
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x, stride = (int64_t)gridDim.x * 256;
  const int64_t n_vec = VEC ? n / 8 * 8 : 0;
  if constexpr (VEC) {
    for (int64_t i = tid * 8; i < n_vec; i += stride * 8) {
      float g[8], m[8];
      load8<GD>(grad, i, g);
      load8<APEXW_F32>(buf, i, m);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (__builtin_isnan(g[j])) g[j] = 0.0f;
        else if (__builtin_isinf(g[j])) g[j] = g[j] > 0.0f ? 65504.0f : -65504.0f;
        m[j] = fmaf(one_minus_mu, g[j], m[j] * mu);
        const float x = rnd<APEXW_BF16>(nesterov ? nesterov_source(g[j], m[j], mu) : m[j]);
        s = fmaf(x, x, s);
      }
      store8<APEXW_F32>(buf, i, m);
    }
  }
  for (int64_t i = n_vec + tid; i < n; i += stride) {
    const float g = muon_grad<GD>(grad, i);
    const float m = fmaf(one_minus_mu, g, APEXW_GLOBAL(float, buf)[i] * mu);
    APEXW_GLOBAL(float, buf)[i] = m;
    const float x = rnd<APEXW_BF16>(nesterov ? nesterov_source(g, m, mu) : m);
    s = fmaf(x, x, s);
  }
  s = wave_sum(s);
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// X = bf16(bf16(buf) / d) with d = bf16(bf16(||bf16(buf)||_F) + eps) (the bf16
// torch ops of zeropower_via_newtonschulz5), written as the work matrix in both
// layouts.  The work matrix is buf itself when rows <= cols, else buf^T.
// 64 x 64 tiles through LDS so both layouts are written with coalesced rows.
template <int GD>
__global__ __launch_bounds__(256) void muon_normalize_kernel(const float* __restrict__ buf, const void* __restrict__ grad,
                                                             int64_t rows, int64_t cols, float mu, int nesterov,
                                                             const float* __restrict__ partial, int n_partial,
                                                             float eps, int tall, uint16_t* __restrict__ x,
                                                             uint16_t* __restrict__ xt, int64_t ldx, int64_t ldxt) {
  __shared__ float red[4];
  __shared__ uint16_t tile[64][66];
  float s = 0.0f;
  for (int i = threadIdx.x; i < n_partial; i += 256) s += partial[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  const float d = rnd<APEXW_BF16>(rnd<APEXW_BF16>(sqrtf(total)) + eps);
  // tile (tr, tc) of buf in its own [rows x cols] layout
  const int64_t tr = (int64_t)blockIdx.y * 64, tc = (int64_t)blockIdx.x * 64;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int r = e >> 6, cidx = e & 63;
    const int64_t gr = tr + r, gc = tc + cidx;
    float v = 0.0f;
    if (gr < rows && gc < cols) {
      const int64_t i = gr * cols + gc;
      float m = APEXW_GLOBAL(const float, buf)[i];
      if (nesterov) m = nesterov_source(muon_grad<GD>(grad, i), m, mu);
      v = rnd<APEXW_BF16>(m) / d;
    }
    tile[r][cidx] = to_bf(v);
  }
  __syncthreads();
  // direct layout D[r][c] = buf-shaped; transposed layout T[c][r]
  uint16_t* direct = tall ? xt : x;
  uint16_t* trans = tall ? x : xt;
  const int64_t ld_direct = tall ? ldxt : ldx, ld_trans = tall ? ldx : ldxt;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int r = e >> 6, cidx = e & 63;
    // direct[tr + r][tc + cidx] = D(tr + r, tc + cidx); trans[tc + r][tr + cidx] = D(tr + cidx, tc + r)
    if (tr + r < rows && tc + cidx < cols) APEXW_GLOBAL(uint16_t, direct)[(tr + r) * ld_direct + tc + cidx] = tile[r][cidx];
    if (tc + r < cols && tr + cidx < rows) APEXW_GLOBAL(uint16_t, trans)[(tc + r) * ld_trans + tr + cidx] = tile[cidx][r];
  }
}

// p = round(round(p * (1 - lr*wd)) + (-lr_eff) * U)   (p.mul_ then p.add_(U, alpha)),
// U read from the NS output in p's [rows x cols] layout (bf16, leading dim ldu).
// VEC: cols % 8 == 0 and 16-byte aligned p / u rows: 8 elements of one row per thread.
template <int PD, bool VEC>
__global__ __launch_bounds__(256) void muon_apply_kernel(void* __restrict__ p, const uint16_t* __restrict__ u,
                                                         int64_t rows, int64_t cols, int64_t ldu, float wd_factor,
                                                         int apply_wd, float neg_lr_eff) {
  const int64_t n = rows * cols;
  if constexpr (VEC) {
    for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += (int64_t)gridDim.x * 256 * 8) {
      const int64_t r = i / cols, c = i - r * cols;
      float x[8], uu[8];
      load8<PD>(p, i, x);
      load8<APEXW_BF16>(u, r * ldu + c, uu);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (apply_wd) x[j] = rnd<PD>(x[j] * wd_factor);
        x[j] = rnd<PD>(fmaf(neg_lr_eff, uu[j], x[j]));
      }
      store8<PD>(p, i, x);
    }
    return;
  }
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / cols, c = i - r * cols;
    float x = load1<PD>(p, i);
    if (apply_wd) x = rnd<PD>(x * wd_factor);
    const float uu = bf(APEXW_GLOBAL(const uint16_t, u)[r * ldu + c]);
    store1<PD>(p, i, rnd<PD>(fmaf(neg_lr_eff, uu, x)));
  }
}

int grid_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return (int)(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

}  // namespace

int apexw_launch_gemm_nt(const uint16_t* a, const uint16_t* b, const uint16_t* et, uint16_t* c, uint16_t* ct,
                         int32_t m, int32_t n, int32_t k, int32_t lda, int32_t ldb, int32_t lde, int32_t ldc,
                         int32_t ldct, int32_t batch, int64_t sa, int64_t sb, int64_t se, int64_t sc, int64_t sct,
                         float alpha, float beta, hipStream_t stream) {
  GemmArgs g{a, b, et, c, ct, sa, sb, se, sc, sct, m, n, k, lda, ldb, lde, ldc, ldct, alpha, beta};
  const int tiles = (m / kBM) * (n / kBN);
  const dim3 grid(((tiles + 7) / 8) * 8, batch);
  const bool add = et && beta != 0.0f;
  if (c && ct) {
    if (add) hipLaunchKernelGGL((gemm_nt_kernel<true, true, true>), grid, dim3(256), 0, stream, g);
    else hipLaunchKernelGGL((gemm_nt_kernel<true, true, false>), grid, dim3(256), 0, stream, g);
  } else if (c) {
    if (add) hipLaunchKernelGGL((gemm_nt_kernel<true, false, true>), grid, dim3(256), 0, stream, g);
    else hipLaunchKernelGGL((gemm_nt_kernel<true, false, false>), grid, dim3(256), 0, stream, g);
  } else {
    if (add) hipLaunchKernelGGL((gemm_nt_kernel<false, true, true>), grid, dim3(256), 0, stream, g);
    else hipLaunchKernelGGL((gemm_nt_kernel<false, true, false>), grid, dim3(256), 0, stream, g);
  }
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

int apexw_launch_gemm_grouped(const apexw_gemm_problem* probs, const uint32_t* items, const int32_t* offsets,
                              int32_t n_wg, int32_t kind, hipStream_t stream) {
  const dim3 grid(n_wg), block(256);
  switch (kind) {
    case APEXW_GEMM_OUT_C:
      hipLaunchKernelGGL((gemm_nt_grouped_kernel<true, false, false>), grid, block, 0, stream, probs, items, offsets);
      break;
    case APEXW_GEMM_OUT_C | APEXW_GEMM_ADD:
      hipLaunchKernelGGL((gemm_nt_grouped_kernel<true, false, true>), grid, block, 0, stream, probs, items, offsets);
      break;
    case APEXW_GEMM_OUT_CT:
      hipLaunchKernelGGL((gemm_nt_grouped_kernel<false, true, false>), grid, block, 0, stream, probs, items, offsets);
      break;
    case APEXW_GEMM_OUT_CT | APEXW_GEMM_ADD:
      hipLaunchKernelGGL((gemm_nt_grouped_kernel<false, true, true>), grid, block, 0, stream, probs, items, offsets);
      break;
    case APEXW_GEMM_OUT_C | APEXW_GEMM_OUT_CT:
      hipLaunchKernelGGL((gemm_nt_grouped_kernel<true, true, false>), grid, block, 0, stream, probs, items, offsets);
      break;
    case APEXW_GEMM_OUT_C | APEXW_GEMM_OUT_CT | APEXW_GEMM_ADD:
      hipLaunchKernelGGL((gemm_nt_grouped_kernel<true, true, true>), grid, block, 0, stream, probs, items, offsets);
      break;
    default:
      return APEXW_ERR_ARG;
  }
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

int apexw_muon_partials(int64_t n) { return grid_for(n) < 1024 ? grid_for(n) : 1024; }

template <int GD>
void launch_prepare(float* buf, const void* g, int64_t rows, int64_t cols, float mu, float one_minus_mu, int nesterov,
                    float eps, uint16_t* x, uint16_t* xt, int64_t ldx, int64_t ldxt, float* partial,
                    hipStream_t stream) {
  const int64_t n = rows * cols;
  const int nb = apexw_muon_partials(n);
  if ((((uintptr_t)buf | (uintptr_t)g) & 15u) == 0)
    hipLaunchKernelGGL((muon_momentum_kernel<GD, true>), dim3(nb), dim3(256), 0, stream, buf, g, n, mu, one_minus_mu,
                       nesterov, partial);
  else
    hipLaunchKernelGGL((muon_momentum_kernel<GD, false>), dim3(nb), dim3(256), 0, stream, buf, g, n, mu, one_minus_mu,
                       nesterov, partial);
  dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
  hipLaunchKernelGGL(muon_normalize_kernel<GD>, grid, dim3(256), 0, stream, buf, g, rows, cols, mu, nesterov, partial,
                     nb, eps, (int)(rows > cols), x, xt, ldx, ldxt);
}

int apexw_launch_muon_prepare(float* buf, const void* g, int32_t g_dtype, int64_t rows, int64_t cols, float mu,
                              float one_minus_mu, int32_t nesterov, float eps, uint16_t* x, uint16_t* xt, int64_t ldx,
                              int64_t ldxt, float* partial, hipStream_t stream) {
  if (g_dtype == APEXW_F32)
    launch_prepare<APEXW_F32>(buf, g, rows, cols, mu, one_minus_mu, nesterov, eps, x, xt, ldx, ldxt, partial, stream);
  else if (g_dtype == APEXW_BF16)
    launch_prepare<APEXW_BF16>(buf, g, rows, cols, mu, one_minus_mu, nesterov, eps, x, xt, ldx, ldxt, partial, stream);
  else
    launch_prepare<APEXW_F16>(buf, g, rows, cols, mu, one_minus_mu, nesterov, eps, x, xt, ldx, ldxt, partial, stream);
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

int apexw_launch_muon_apply(void* p, int32_t p_dtype, const uint16_t* u, int64_t rows, int64_t cols, int64_t ldu,
                            float wd_factor, int32_t apply_wd, float neg_lr_eff, hipStream_t stream) {
  const int64_t n = rows * cols;
  const bool vec = cols % 8 == 0 && ldu % 8 == 0 && (((uintptr_t)p | (uintptr_t)u) & 15u) == 0;
  const dim3 grid(grid_for(vec ? n / 8 : n));
  if (p_dtype == APEXW_F32) {
    if (vec) hipLaunchKernelGGL((muon_apply_kernel<APEXW_F32, true>), grid, dim3(256), 0, stream, p, u, rows, cols, ldu,
                                wd_factor, apply_wd, neg_lr_eff);
    else hipLaunchKernelGGL((muon_apply_kernel<APEXW_F32, false>), grid, dim3(256), 0, stream, p, u, rows, cols, ldu,
                            wd_factor, apply_wd, neg_lr_eff);
  } else if (p_dtype == APEXW_BF16) {
    if (vec) hipLaunchKernelGGL((muon_apply_kernel<APEXW_BF16, true>), grid, dim3(256), 0, stream, p, u, rows, cols,
                                ldu, wd_factor, apply_wd, neg_lr_eff);
    else hipLaunchKernelGGL((muon_apply_kernel<APEXW_BF16, false>), grid, dim3(256), 0, stream, p, u, rows, cols, ldu,
                            wd_factor, apply_wd, neg_lr_eff);
  } else {
    if (vec) hipLaunchKernelGGL((muon_apply_kernel<APEXW_F16, true>), grid, dim3(256), 0, stream, p, u, rows, cols, ldu,
                                wd_factor, apply_wd, neg_lr_eff);
    else hipLaunchKernelGGL((muon_apply_kernel<APEXW_F16, false>), grid, dim3(256), 0, stream, p, u, rows, cols, ldu,
                            wd_factor, apply_wd, neg_lr_eff);
  }
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}
