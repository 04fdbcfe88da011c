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
#include <type_traits>

#include "common.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) uint16_t u16x4;
typedef __attribute__((ext_vector_type(4))) short v4i16;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

constexpr int kBM = 256, kBN = 256;
// K is staged through LDS 32 at a time in kStages rotating buffers of 32 KB
// (A then B, each [256 rows x 32] bf16 with 64-byte rows): 160 KB, all of a
// CU's LDS.  The four 16-byte chunks of row r are stored XOR-swizzled (chunk c
// at slot c ^ ((r / 4) % 4)), so the fragment reads of 16 consecutive rows
// cover all 64 banks once.
constexpr int kBK = 32, kStages = 5;
APEXW_DEV int lds_off(int row, int chunk) { return row * kBK + ((chunk ^ ((row >> 2) & 3)) << 3); }

// Element offset of (r, c) in a matrix with ld columns, row-major or in 32 x 32
// panels (APEXW_GEMM_PANEL: panel (r / 32, c / 32) is 1024 contiguous elements,
// row-major inside, panels in row-major order).  For r and c multiples of 32 the
// offsets of the two layouts differ only in the column term, and offsets add:
// poff(r0 + r, c0 + c) = poff(r0, c0) + poff(r, c).
APEXW_DEV uint32_t poff(int r, int c, int ld, bool panel) {
  return panel ? (uint32_t)((r >> 5) * 32 * ld + ((c >> 5) << 10) + ((r & 31) << 5) + (c & 31))
               : (uint32_t)(r * ld + c);
}
// the same for whole matrices (64-bit offsets)
APEXW_DEV int64_t poff64(int64_t r, int64_t c, int64_t ld, bool panel) {
  return panel ? (r >> 5) * 32 * ld + ((c >> 5) << 10) + ((r & 31) << 5) + (c & 31) : r * ld + c;
}

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

typedef uint16_t LdsStage[2][kBM * kBK];   // [A | B][256 x 32]

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

// s_waitcnt vmcnt(n) for the n the K loop needs (an immediate operand).
// Counts are multiples of the copies per stage (8, or 6 for half tiles); any
// other n waits for the next lower listed count, which is also correct.
APEXW_DEV void wait_vm(int n) {
  if (n >= 32) asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
  else if (n >= 24) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
  else if (n >= 18) asm volatile("s_waitcnt vmcnt(18)" ::: "memory");
  else if (n >= 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  else if (n >= 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  else if (n >= 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else if (n >= 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// The Muon update fused into the X' epilogue (APEXW_GEMM_APPLY): p [rows x
// cols] row-major, O = p (or p^T when transposed) in the tile's coordinates;
// row0 / col0 are the tile's origin in O.  p == nullptr: no update.
struct ApplyArgs {
  void* p;
  int64_t rows, cols, row0, col0;
  float wd_factor, neg_lr;
  int dtype;
  bool transposed, wd, vec;
};

// x = p; with decay x = rnd(x * wd_factor); p = rnd(x + neg_lr * u), for the
// cnt (<= 8) consecutive elements of p from index i (the element order of
// apexw/muon.py:852-858's p.mul_ then p.add_, as muon_apply_kernel does it)
template <int PD>
APEXW_DEV void apply_run(const ApplyArgs& ap, int64_t i, const float (&u)[8], int cnt) {
  if (ap.vec && cnt == 8) {
    float x[8];
    load8<PD>(ap.p, i, x);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      if (ap.wd) x[t] = rnd<PD>(x[t] * ap.wd_factor);
      x[t] = rnd<PD>(fmaf(ap.neg_lr, u[t], x[t]));
    }
    store8<PD>(ap.p, i, x);
    return;
  }
  for (int t = 0; t < cnt; ++t) {
    float x = load1<PD>(ap.p, i + t);
    if (ap.wd) x = rnd<PD>(x * ap.wd_factor);
    store1<PD>(ap.p, i + t, rnd<PD>(fmaf(ap.neg_lr, u[t], x)));
  }
}

// One output tile: O = alpha * A B^T + beta * E (bf16 in, fp32 accumulate,
// bf16 out, round to nearest even), 256 x 256, or 128 x 256 with kHalf (the
// split tail tiles of a grouped launch).  A and B point at the tile's first row
// of each operand; Et, C and Ct at the tile's origin in their own layouts.  256
// threads = 4 waves in a 2 x 2 arrangement, each owning a kWM x 128 block
// (kWM = 128, or 64 with kHalf) as (kWM / 32) x 4 MFMA 32x32x16 accumulators.
// Template flags select the epilogue: write O row-major (kC), transposed (kCt,
// skipped at run time when write_ct is false), add beta * E (kAdd).
//
// K pipeline.  Stage h = K columns [32 h, 32 h + 32), buffer h % 5, two MFMA
// k-steps (a, b) whose fragments sit in register slots 0 and 1.  Iteration h:
//   1. the MFMAs of step h.a, each of the first kFrags followed by one LDS read
//      of step h.b's fragments (slot 1, free since the MFMAs of step (h-1).b
//      were issued);
//   2. wait until stage h + 1's copies have landed and this wave's LDS reads
//      have returned, then barrier;
//   3. the MFMAs of step h.b, the first kFrags each followed by one LDS read of
//      step (h+1).a (slot 0), and the kCopies global -> LDS copies of stage
//      h + 5 into buffer h % 5 spread evenly over them (one after every other
//      MFMA: issued in a burst, the copies stall the wave's in-order issue on a
//      full memory pipeline, and with one wave per SIMD the matrix core idles).
// Stage h + 1 is read only after the barrier in 2 that follows its wait, and
// buffer h % 5 is refilled only after that barrier, which every wave reaches
// after its last reads of stage h.  A stage's copies have about three and a
// half iterations to land.
//
// kNN: B is given as [K x N] row-major (O = alpha A B + beta E) instead of
// [N x K].  Its LDS stage is then 32 K rows x 256 columns, and each B fragment
// (8 consecutive k of one column) is assembled by two transposing LDS reads
// (ds_read_b64_tr_b16: in each group of 16 lanes, lane 4 r + c receives
// element c of the 8-byte rows addressed by lanes r, r + 4, r + 8, r + 12).
//
// Addend on the matrix cores (diag_k0 >= 0): when E is the B operand itself
// read at K = diag_k0 + i (E[i][j] = B[j][diag_k0 + i], or B[diag_k0 + i][j]
// for kNN, as in X' = B X + a X) and alpha == 1, the B fragments of K
// [diag_k0, diag_k0 + rows) are exactly the addend.  There each wave adds
// beta E with extra MFMAs against a one-hot fragment holding beta on the
// diagonal (beta split into two bf16 parts, hi + lo, within 2^-18 of beta), so
// the epilogue reads no addend.
template <bool kC, bool kCt, bool kAdd, bool kNN, bool kHalf, bool kPanel>
APEXW_DEV void gemm_tile(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, int32_t lda, int32_t ldb,
                         int32_t k, const uint16_t* __restrict__ Et, int32_t lde, uint16_t* __restrict__ C,
                         int32_t ldc, uint16_t* __restrict__ Ct, int32_t ldct, bool write_ct, float alpha,
                         float beta, int32_t diag_k0, const ApplyArgs& ap, LdsStage* lds) {
  constexpr bool panel = kPanel;   // operands and outputs in 32 x 32 panels (APEXW_GEMM_PANEL)
  constexpr int kWM = kHalf ? 64 : 128;   // rows of a wave's block
  constexpr int kFA = kWM / 32;           // A fragments (32-row blocks) per wave and k-step
  constexpr int kACopies = kWM / 32;      // A copy instructions per wave and stage (16 rows each, 4 waves)
  constexpr int kCopies = kACopies + 4;   // per stage and wave: A, then the 4 of B
  constexpr int kFrags = kFA + 4;         // fragment reads per k-step
  constexpr int kMM = kFA * 4;            // MFMAs per k-step
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Copies: each wave instruction fills 1 KB of LDS, lane L landing at byte
  // 16 L.  [rows x K] operands: 16 rows of 64 bytes, lane L at row 16 q + L / 4,
  // slot L % 4, which holds column chunk (L % 4) ^ ((L / 16) % 4).  kNN B: 2 K
  // rows of 512 bytes, lane L at row 2 q + L / 32, slot L % 32, holding column
  // chunk (L % 32) ^ (4 (row % 4)) (so the transposing reads of 4 consecutive
  // rows hit distinct banks).  A stage is 16 instructions for B and 16 (8 with
  // kHalf) for A; wave w issues q = kACopies w .. of A and 4 w .. 4 w + 3 of B.
  // With panels a [rows x K] stage of 16 rows is 1 KB of one panel, contiguous,
  // and a [K x N] stage row band is 8 consecutive panels: full 128-byte lines.
  uint32_t goff[kCopies];
#pragma unroll
  for (int i = 0; i < kACopies; ++i) {
    const int row = 16 * (kACopies * wave + i) + (lane >> 2), chunk = (lane & 3) ^ ((lane >> 4) & 3);
    goff[i] = poff(row, chunk * 8, lda, panel) * 2u;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (kNN) {
      const int krow = 2 * (4 * wave + i) + (lane >> 5), nchunk = (lane & 31) ^ (4 * (krow & 3));
      goff[kACopies + i] = poff(krow, nchunk * 8, ldb, panel) * 2u;
    } else {
      const int row = 16 * (4 * wave + i) + (lane >> 2), chunk = (lane & 3) ^ ((lane >> 4) & 3);
      goff[kACopies + i] = poff(row, chunk * 8, ldb, panel) * 2u;
    }
  }
  // LDS byte addresses of this wave's first A and B chunks in stage 0 (wave-uniform)
  const uint32_t ldsA0 = __builtin_amdgcn_readfirstlane(lds_address(&lds[0][0][kACopies * wave * 512]));
  const uint32_t ldsB0 = __builtin_amdgcn_readfirstlane(lds_address(&lds[0][1][4 * wave * 512]));
  constexpr uint32_t kStageBytes = sizeof(LdsStage), kChunk = 1024;
  const uint16_t* A_s = uniform_ptr(A);
  const uint16_t* B_s = uniform_ptr(B);
  // elements from one K stage to the next along a [rows x K] operand: the next
  // 32 columns, or the next panel; a [K x N] operand moves 32 rows in both layouts
  const int kstep = panel ? 1024 : kBK;
  // copy i (0 .. kCopies - 1) of stage h: A chunks, then B chunks 0..3
  auto copy = [&](int h, int i) {
    const uint32_t st = (uint32_t)(h % kStages) * kStageBytes;
    if (i < kACopies) lds_copy16(ldsA0 + st + i * kChunk, goff[i], A_s + (int64_t)h * kstep);
    else lds_copy16(ldsB0 + st + (i - kACopies) * kChunk, goff[i],
                    B_s + (kNN ? (int64_t)h * kBK * ldb : (int64_t)h * kstep));
  };

  f32x16 acc[kFA][4];
#pragma unroll
  for (int a = 0; a < kFA; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f32x16{};

  // MFMA 32x32x16 operand layout: lane l supplies row (l % 32) and k = 8 (l / 32) .. +7.
  const int frag_row = lane & 31, frag_c = lane >> 5;
  bf16x8 fa[2][kFA], fb[2][4];
  // fragment read i (0 .. kFrags - 1) of k-step s of stage h: A fragments, then B 0..3
  auto frag = [&](int h, int s, int i) {
    const uint16_t* st = lds[h % kStages][i < kFA ? 0 : 1];
    if (kNN && i >= kFA) {
      // lane l = 16 g + 4 r + j' of group g addresses K row 16 s + 8 (g / 2) + j'
      // (+ 4 for the upper half), columns n .. n + 3 with n = 16 (g % 2) + 4 r
      // of the 32-column block; it receives column 16 (g % 2) + (l % 16) = l % 32
      // at 4 consecutive K rows, i.e. the MFMA B layout
      const int g = lane >> 4, r = lane & 3, jr = (lane >> 2) & 3;
      const int n = wn * 128 + (i - kFA) * 32 + 16 * (g & 1) + 4 * r;
      const int k0 = 16 * s + 8 * (g >> 1) + jr;   // k0 % 4 == jr, as for k0 + 4
      const int slot = (n >> 3) ^ (4 * jr);
      const int e0 = k0 * 256 + slot * 8 + (n & 7), e1 = e0 + 4 * 256;
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)&st[e0]);
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)&st[e1]);
      const u32x2 wl = __builtin_bit_cast(u32x2, lo), wh = __builtin_bit_cast(u32x2, hi);
      fb[s][i - kFA] = __builtin_bit_cast(bf16x8, u32x4{wl[0], wl[1], wh[0], wh[1]});
      return;
    }
    const int row = (i < kFA ? wm * kWM + i * 32 : wn * 128 + (i - kFA) * 32) + frag_row;
    const bf16x8 v = *(const bf16x8*)&st[lds_off(row, s * 2 + frag_c)];
    if (i < kFA) fa[s][i] = v;
    else fb[s][i - kFA] = v;
  };
  // the kMM MFMAs of slot s, side(j) issued after MFMA j; sched_barrier(0)
  // fences keep that interleaving (the scheduler would otherwise cluster the
  // reads next to their first use and expose the LDS latency)
  auto mma = [&](int s, auto&& side) {
#pragma unroll
    for (int j = 0; j < kMM; ++j) {
      acc[j >> 2][j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[s][j >> 2], fb[s][j & 3], acc[j >> 2][j & 3], 0,
                                                                    0, 0);
      __builtin_amdgcn_sched_barrier(0);
      side(j);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // beta E on the matrix cores (see above): stage h holds K columns
  // [32 h, 32 h + 32), i.e. rows 32 h - diag_k0 .. + 31 of the addend, which
  // fall in this wave's A block (32 h - diag_k0 - kWM wm) / 32 when in range
  const bool diag = kAdd && diag_k0 >= 0;
  const uint32_t beta_hi = f32_to_bf16_bits(beta);
  const uint32_t beta_lo = f32_to_bf16_bits(beta - __uint_as_float(beta_hi << 16));
  auto diag_mma = [&](int h, int s) {
    const int rel = h * kBK - (diag_k0 + wm * kWM);
    if (rel < 0 || rel >= kWM) return;
    // lane l feeds row l % 32 of the block and k = 16 s + 8 (l / 32) + t: the
    // diagonal element sits at t = l % 32 - 16 s - 8 (l / 32)
    const int t = (lane & 31) - 16 * s - 8 * (lane >> 5);
    u32x4 dh = {0u, 0u, 0u, 0u}, dl = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const bool hit = (t >> 1) == w && t >= 0 && t < 8;
      const uint32_t sh = (uint32_t)(t & 1) * 16u;
      dh[w] = hit ? beta_hi << sh : 0u;
      dl[w] = hit ? beta_lo << sh : 0u;
    }
    const bf16x8 fh = __builtin_bit_cast(bf16x8, dh), fl = __builtin_bit_cast(bf16x8, dl);
    auto add = [&](auto blk_c) {
      constexpr int blk = decltype(blk_c)::value;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        acc[blk][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fh, fb[s][b], acc[blk][b], 0, 0, 0);
        acc[blk][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fl, fb[s][b], acc[blk][b], 0, 0, 0);
      }
    };
    if constexpr (kFA == 4) {
      switch (rel >> 5) {
        case 0: add(std::integral_constant<int, 0>()); break;
        case 1: add(std::integral_constant<int, 1>()); break;
        case 2: add(std::integral_constant<int, 2>()); break;
        default: add(std::integral_constant<int, 3>()); break;
      }
    } else {
      if ((rel >> 5) == 0) add(std::integral_constant<int, 0>());
      else add(std::integral_constant<int, 1>());
    }
  };
  // lgkmcnt(0) through the builtin (vmcnt and expcnt fields at their no-wait
  // maxima), so the compiler knows this wave's LDS reads have returned and adds
  // no later waits for them; the barrier itself is asm with a memory clobber so
  // no LDS access moves across it
  auto barrier = [&]() {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("s_barrier" ::: "memory");
  };

  const int n = k / kBK;
  const int first = n < kStages ? n : kStages;
  for (int h = 0; h < first; ++h)
#pragma unroll
    for (int i = 0; i < kCopies; ++i) copy(h, i);
  wait_vm(kCopies * (first - 1));   // stage 0 landed
  barrier();
#pragma unroll
  for (int i = 0; i < kFrags; ++i) frag(0, 0, i);
  // one iteration; kNext: a stage h + 1 exists, kRefill: a stage h + 5 exists
  auto iteration = [&](int h, auto next_c, auto refill_c) {
    constexpr bool kNext = decltype(next_c)::value, kRefill = decltype(refill_c)::value;
    mma(0, [&](int j) {
      if (j < kFrags) frag(h, 1, j);
    });
    if (diag) diag_mma(h, 0);
    // stage h + 1 landed; copies of the stages after it may still be in flight
    const int last_issued = (h + kStages - 1 < n ? h + kStages - 1 : n - 1);
    wait_vm(kNext ? kCopies * (last_issued - (h + 1)) : 0);
    barrier();
    mma(1, [&](int j) {
      if constexpr (kNext) {
        if (j < kFrags) frag(h + 1, 0, j);
      }
      if constexpr (kRefill) {
        if ((j * kCopies) / kMM != ((j + 1) * kCopies) / kMM) copy(h + kStages, (j * kCopies) / kMM);
      }
    });
    if (diag) diag_mma(h, 1);
  };
  typedef std::integral_constant<bool, true> yes;
  typedef std::integral_constant<bool, false> no;
  int h = 0;
  for (; h + kStages < n; ++h) iteration(h, yes(), yes());
  for (; h + 1 < n; ++h) iteration(h, yes(), no());
  iteration(h, no(), no());   // n >= 1: the last stage

  // Epilogue.  Accumulator register r of lane l holds row 8 (r / 4) + 4 (l / 32) + r % 4,
  // column l % 32 of its 32 x 32 block: four consecutive rows of one column per group.
  // After the last barrier the operand tiles are dead: each wave stages its
  // kWM x 128 block of O in its own 32 KB of LDS, then writes it row by row to C
  // and column by column to Ct, both as 16-byte stores along output rows.  The
  // stage keeps 16-byte chunks XOR-swizzled by row / 8 so that the row reads
  // (16 lanes per row) and the column reads (lanes down a column) each hit
  // distinct banks.  A wave reads back only what it wrote itself, and LDS keeps
  // one wave's accesses in order, so no barrier is needed.
  uint16_t* stage = lds[wave][0];   // 32 KB per wave
  auto swz = [](int r, int c) { return r * 128 + ((((c >> 3) ^ (r >> 3)) & 15) << 3) + (c & 7); };
  const int il0 = (lane >> 5) * 4, jl0 = lane & 31;           // within the wave's block
  const int gi0 = wm * kWM + il0, gj0 = wn * 128 + jl0;       // within the tile
#pragma unroll
  for (int a = 0; a < kFA; ++a) {
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
          if (!diag) {
            const u16x4 e = *APEXW_GLOBAL(const u16x4, Et + poff(gj0 + b * 32, gi0 + a * 32 + q * 8, lde, panel));
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = fmaf(beta, bf(e[r]), v[r]);
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) stage[swz(il + r, jl)] = to_bf(v[r]);
      }
    }
  }
  if constexpr (kC) {
    if (ap.p) {
      // the wave's block of O in O coordinates; p elements outside p's shape
      // (the zero padding of the work matrix) are skipped
      const int64_t gr0 = ap.row0 + wm * kWM, gc0 = ap.col0 + wn * 128;
      auto upd = [&](auto pd_c) {
        constexpr int PD = decltype(pd_c)::value;
        if (!ap.transposed) {
          // row by row: lane chunk = 8 consecutive elements of one row of p
          for (int it = 0; it < kWM / 4; ++it) {
            const int c = it * 64 + lane, r = c >> 4, c16 = c & 15;
            const int64_t gi = gr0 + r, gj = gc0 + c16 * 8;
            if (gi >= ap.rows || gj >= ap.cols) continue;
            const u32x4 v = *(const u32x4*)&stage[swz(r, c16 * 8)];
            float u[8];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              u[2 * t] = bf((uint16_t)(v[t] & 0xFFFFu));
              u[2 * t + 1] = bf((uint16_t)(v[t] >> 16));
            }
            apply_run<PD>(ap, gi * ap.cols + gj, u, (int)min<int64_t>(8, ap.cols - gj));
          }
        } else {
          // column by column of the block = row by row of p: p[gc0 + jl][gr0 + il + t] = O[gr0 + il + t][gc0 + jl]
          constexpr int kPerRow = kWM / 8;
          for (int it = 0; it < kWM / 4; ++it) {
            const int c = it * 64 + lane, jl = c / kPerRow, il = (c % kPerRow) * 8;
            const int64_t prow = gc0 + jl, pcol = gr0 + il;
            if (prow >= ap.rows || pcol >= ap.cols) continue;
            float u[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) u[t] = bf(stage[swz(il + t, jl)]);
            apply_run<PD>(ap, prow * ap.cols + pcol, u, (int)min<int64_t>(8, ap.cols - pcol));
          }
        }
      };
      if (ap.dtype == APEXW_F32) upd(std::integral_constant<int, APEXW_F32>());
      else if (ap.dtype == APEXW_BF16) upd(std::integral_constant<int, APEXW_BF16>());
      else upd(std::integral_constant<int, APEXW_F16>());
    }
    if (C) {
#pragma unroll 4
      for (int it = 0; it < kWM / 4; ++it) {
        const int c = it * 64 + lane, r = c >> 4, c16 = c & 15;
        const u32x4 v = *(const u32x4*)&stage[swz(r, c16 * 8)];
        __builtin_nontemporal_store(v, APEXW_GLOBAL(u32x4, C + poff(wm * kWM + r, wn * 128 + c16 * 8, ldc, panel)));
      }
    }
  }
  if constexpr (kCt) {
    if (write_ct) {
      constexpr int kPerRow = kWM / 8;   // 16-byte chunks per Ct row of the block
#pragma unroll 2
      for (int it = 0; it < kWM / 4; ++it) {
        // Ct row jl (= column jl of the block), elements il .. il + 7
        const int c = it * 64 + lane, jl = c / kPerRow, il = (c % kPerRow) * 8;
        u32x4 v;
#pragma unroll
        for (int t = 0; t < 4; ++t)
          v[t] = (uint32_t)stage[swz(il + 2 * t, jl)] | ((uint32_t)stage[swz(il + 2 * t + 1, jl)] << 16);
        *APEXW_GLOBAL(u32x4, Ct + poff(wn * 128 + jl, wm * kWM + il, ldct, panel)) = v;
      }
    }
  }
}

// Batched GEMM over one shape: one workgroup per output tile, blockIdx.y = batch entry.
template <bool kC, bool kCt, bool kAdd>
__global__ __launch_bounds__(256, 1) void gemm_nt_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) LdsStage lds[kStages];

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
  gemm_tile<kC, kCt, kAdd, false, false, false>(
      g.a + batch * g.sa + row0 * g.lda, g.b + batch * g.sb + col0 * g.ldb, g.lda, g.ldb, g.k,
      kAdd ? g.et + batch * g.se + col0 * g.lde + row0 : nullptr, g.lde,
      kC ? g.c + batch * g.sc + row0 * g.ldc + col0 : nullptr, g.ldc,
      kCt ? g.ct + batch * g.sct + col0 * g.ldct + row0 : nullptr, g.ldct, true, g.alpha, g.beta, -1, ApplyArgs{}, lds);
}

// Grouped GEMM: every problem of a launch (different shapes, K and operands)
// in one grid, one workgroup per output tile.  The tiles are split into
// kQueues queues, one per XCD: workgroups are dispatched round-robin over the
// 8 XCDs, so workgroup b runs on XCD b % 8 and computes tile b / 8 of queue
// b % 8.  Each XCD thus works through its own queue in order, a new workgroup
// starting on whichever of its CUs frees first; a queue is one contiguous band
// of tiles in locality order, longest first.  Workgroups past the end of their
// queue exit at once.  An item packs (problem << 24) | (part << 22) |
// (tile row << 11) | tile column, part 0 for a whole 256 x 256 tile and 1 / 2
// for its upper / lower 128-row half (the tail of a queue may be split so that
// its last round fills the XCD).  A symmetric problem (APEXW_GEMM_SYM) lists
// only tiles with row <= column and mirrors each off-diagonal tile through the
// transposed store (ct == c).
constexpr int kQueues = APEXW_GEMM_QUEUES;

template <bool kC, bool kCt, bool kAdd, bool kNN, bool kPanel>
__global__ __launch_bounds__(256, 1) void gemm_nt_grouped_kernel(const apexw_gemm_problem* __restrict__ probs,
                                                                 const uint32_t* __restrict__ items,
                                                                 const int32_t* __restrict__ queue_offsets,
                                                                 const apexw_amp_dyn* __restrict__ amp) {
  __shared__ __attribute__((aligned(16))) LdsStage lds[kStages];
  if (amp && amp->skip) return;   // GradScaler found an inf / NaN: no product, no update
  const int q = (int)(blockIdx.x % kQueues), i = (int)(blockIdx.x / kQueues);
  const int begin = queue_offsets[q];
  if (i >= queue_offsets[q + 1] - begin) return;
  const uint32_t code = items[begin + i];
  const apexw_gemm_problem& p = probs[code >> 24];
  const int part = (int)((code >> 22) & 3u);
  const int tm = (int)((code >> 11) & 0x7ffu), tn = (int)(code & 0x7ffu);
  const int64_t row0 = (int64_t)tm * kBM + (part == 2 ? kBM / 2 : 0), col0 = (int64_t)tn * kBN;
  const bool mirror = !(p.flags & APEXW_GEMM_SYM) || tm != tn;
  // APEXW_GEMM_ADD_B: the addend is the B operand read at K = row0 + i,
  // accumulated on the matrix cores (validated: alpha == 1, m <= k, no et)
  const bool diag = kAdd && (p.flags & APEXW_GEMM_ADD_B);
  // tile origins are multiples of 32: with panels only the column term of a
  // base offset changes (column c0 starts panel column c0 / 32, c0 * 32 elements in)
  const int64_t cs = kPanel ? 32 : 1;
  const uint16_t* A = (const uint16_t*)p.a + row0 * p.lda;
  const uint16_t* B = (const uint16_t*)p.b + (kNN ? col0 * cs : col0 * p.ldb);
  const uint16_t* Et = kAdd && !diag ? (const uint16_t*)p.et + col0 * p.lde + row0 * cs : nullptr;
  uint16_t* C = kC && p.c ? (uint16_t*)p.c + row0 * p.ldc + col0 * cs : nullptr;
  uint16_t* Ct = kCt ? (uint16_t*)p.ct + col0 * p.ldct + row0 * cs : nullptr;
  const int32_t dk = diag ? (int32_t)row0 : -1;
  ApplyArgs ap{};
  if (kC && (p.flags & APEXW_GEMM_APPLY)) {
    ap.p = p.p;
    ap.rows = p.p_rows;
    ap.cols = p.p_cols;
    ap.row0 = row0;
    ap.col0 = col0;
    ap.wd_factor = p.wd_factor;
    ap.neg_lr = p.neg_lr;
    ap.dtype = p.p_dtype;
    ap.transposed = (p.flags & APEXW_GEMM_APPLY_T) != 0;
    ap.wd = (p.flags & APEXW_GEMM_APPLY_WD) != 0;
    ap.vec = p.p_cols % 8 == 0 && ((uintptr_t)p.p & 15u) == 0;
  }
  if (part)
    gemm_tile<kC, kCt, kAdd, kNN, true, kPanel>(A, B, p.lda, p.ldb, p.k, Et, p.lde, C, p.ldc, Ct, p.ldct, mirror,
                                                p.alpha, p.beta, dk, ap, lds);
  else
    gemm_tile<kC, kCt, kAdd, kNN, false, kPanel>(A, B, p.lda, p.ldb, p.k, Et, p.lde, C, p.ldc, Ct, p.ldct, mirror,
                                                 p.alpha, p.beta, dk, ap, lds);
}

// ---------------------------------------------------------------------------
// Momentum (apexw/muon.py:763-792, fp32 buffer): buf = buf * mu, then
// buf += (1 - mu) * g with g sanitized (NaN -> 0, +-Inf -> +-65504) and widened
// to fp32.  The NS input ("update source") is buf, or lerp(g, buf, mu) with
// Nesterov.  Per-block partial sums of squares of bf16(update source) give the
// Frobenius norm of the bf16 work matrix.
// ---------------------------------------------------------------------------
// the reference unscales p.grad in place (grad dtype) before the step
// (apexw/muon.py:566-590), then the momentum update sanitizes it
template <int GD> APEXW_DEV float muon_grad(const void* grad, int64_t i, float inv) {
  float g = load1<GD>(grad, i);
  if (inv != 1.0f) g = rnd<GD>(g * inv);
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
                                                            float inv, float* __restrict__ partial,
                                                            const apexw_amp_dyn* __restrict__ amp) {
  if (amp) {
    if (amp->skip) return;
    inv = amp->grad_inv_scale;
  }
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
        if (inv != 1.0f) g[j] = rnd<GD>(g[j] * inv);
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
    const float g = muon_grad<GD>(grad, i, inv);
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
// orientations.  The work matrix is buf itself when rows <= cols, else buf^T.
// 64 x 64 tiles through LDS so both are written along their rows; panel: the
// outputs are stored in 32 x 32 panels (the grouped GEMM's APEXW_GEMM_PANEL).
template <int GD>
__global__ __launch_bounds__(256) void muon_normalize_kernel(const float* __restrict__ buf, const void* __restrict__ grad,
                                                             int64_t rows, int64_t cols, float mu, int nesterov,
                                                             float inv, const float* __restrict__ partial, int n_partial,
                                                             float eps, int tall, uint16_t* __restrict__ x,
                                                             uint16_t* __restrict__ xt, int64_t ldx, int64_t ldxt,
                                                             bool panel, const apexw_amp_dyn* __restrict__ amp) {
  __shared__ float red[4];
  __shared__ uint16_t tile[64][66];
  if (amp) {
    if (amp->skip) return;
    inv = amp->grad_inv_scale;
  }
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
      if (nesterov) m = nesterov_source(muon_grad<GD>(grad, i, inv), m, mu);
      v = rnd<APEXW_BF16>(m) / d;
    }
    tile[r][cidx] = to_bf(v);
  }
  __syncthreads();
  // direct layout D[r][c] = buf-shaped; transposed layout T[c][r]; xt may be
  // null (only the wide work matrix is wanted)
  uint16_t* direct = tall ? xt : x;
  uint16_t* trans = tall ? x : xt;
  const int64_t ld_direct = tall ? ldxt : ldx, ld_trans = tall ? ldx : ldxt;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int r = e >> 6, cidx = e & 63;
    // direct[tr + r][tc + cidx] = D(tr + r, tc + cidx); trans[tc + r][tr + cidx] = D(tr + cidx, tc + r)
    if (direct && tr + r < rows && tc + cidx < cols)
      APEXW_GLOBAL(uint16_t, direct)[poff64(tr + r, tc + cidx, ld_direct, panel)] = tile[r][cidx];
    if (trans && tc + r < cols && tr + cidx < rows)
      APEXW_GLOBAL(uint16_t, trans)[poff64(tc + r, tr + cidx, ld_trans, panel)] = tile[cidx][r];
  }
}

// p = round(round(p * (1 - lr*wd)) + (-lr_eff) * U)   (p.mul_ then p.add_(U, alpha)),
// U read from the NS output in p's [rows x cols] layout (bf16, leading dim ldu).
// VEC: cols % 8 == 0 and 16-byte aligned p / u rows: 8 elements of one row per thread.
// panel: U stored in 32 x 32 panels (APEXW_GEMM_PANEL); 8 consecutive elements of
// a row starting at a multiple of 8 stay inside one panel row.
template <int PD, bool VEC>
__global__ __launch_bounds__(256) void muon_apply_kernel(void* __restrict__ p, const uint16_t* __restrict__ u,
                                                         int64_t rows, int64_t cols, int64_t ldu, bool panel,
                                                         float wd_factor, int apply_wd, float neg_lr_eff,
                                                         const apexw_amp_dyn* __restrict__ amp) {
  if (amp && amp->skip) return;
  const int64_t n = rows * cols;
  if constexpr (VEC) {
    for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += (int64_t)gridDim.x * 256 * 8) {
      const int64_t r = i / cols, c = i - r * cols;
      float x[8], uu[8];
      load8<PD>(p, i, x);
      load8<APEXW_BF16>(u, poff64(r, c, ldu, panel), uu);
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
    const float uu = bf(APEXW_GLOBAL(const uint16_t, u)[poff64(r, c, ldu, panel)]);
    store1<PD>(p, i, rnd<PD>(fmaf(neg_lr_eff, uu, x)));
  }
}

// The same update with U given transposed, u[c * ldu + r] = U[r][c] (the wide
// work matrix of a tall parameter): 64 x 64 tiles through LDS, so both U and p
// are read and written along their rows.
template <int PD>
__global__ __launch_bounds__(256) void muon_apply_t_kernel(void* __restrict__ p, const uint16_t* __restrict__ u,
                                                           int64_t rows, int64_t cols, int64_t ldu, bool panel,
                                                           float wd_factor, int apply_wd, float neg_lr_eff,
                                                           const apexw_amp_dyn* __restrict__ amp) {
  __shared__ uint16_t tile[64][66];
  if (amp && amp->skip) return;
  const int64_t tr = (int64_t)blockIdx.y * 64, tc = (int64_t)blockIdx.x * 64;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int cc = e >> 6, rr = e & 63;
    if (tc + cc < cols && tr + rr < rows)
      tile[cc][rr] = APEXW_GLOBAL(const uint16_t, u)[poff64(tc + cc, tr + rr, ldu, panel)];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int rr = e >> 6, cc = e & 63;
    if (tr + rr < rows && tc + cc < cols) {
      const int64_t i = (tr + rr) * cols + tc + cc;
      float x = load1<PD>(p, i);
      if (apply_wd) x = rnd<PD>(x * wd_factor);
      store1<PD>(p, i, rnd<PD>(fmaf(neg_lr_eff, bf(tile[cc][rr]), x)));
    }
  }
}

int grid_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return (int)(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

}  // namespace

// Coordinate-wise update of a Muon parameter with a dimension under 16 (or a
// vector): the reference's fallback in ApexMuon._step_single
// (apexw/muon.py:775-799, :841-858).  One workgroup per tensor:
//   g = nan_to_num(dtype_round(g * inv)); buf = buf * mu + (1 - mu) g;
//   s = buf (or lerp(g, buf, mu) with nesterov);
//   U = s / (std(s, unbiased=False) + 1e-7)   (numel 1: s / (|s| + 1e-7));
//   p = dtype_round(p * wd_factor) (with decay); p = dtype_round(p + neg_lr * dtype_round(U)).
// mean and variance are two passes over the tensor, each a workgroup reduction.
constexpr int kCwThreads = 1024;

APEXW_DEV float block_sum_cw(float x, float* red) {
  x = wave_sum(x);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = x;
  __syncthreads();
  float t = 0.0f;
  for (int i = 0; i < nw; ++i) t += red[i];
  __syncthreads();
  return t;
}

template <int GD, int PD>
__global__ __launch_bounds__(kCwThreads) void muon_coordwise_kernel(float* __restrict__ buf, const void* __restrict__ grad,
                                                                    void* __restrict__ p, int64_t n, float mu,
                                                                    float one_minus_mu, int nesterov, float inv,
                                                                    float wd_factor, int apply_wd, float neg_lr,
                                                                    const apexw_amp_dyn* __restrict__ amp) {
  __shared__ float red[kCwThreads / 64];
  if (amp) {
    if (amp->skip) return;
    inv = amp->grad_inv_scale;
  }
  const int64_t tid = threadIdx.x, stride = blockDim.x;
  float sum = 0.0f;
  for (int64_t i = tid; i < n; i += stride) {
    const float g = muon_grad<GD>(grad, i, inv);
    const float m = fmaf(one_minus_mu, g, buf[i] * mu);
    buf[i] = m;
    sum += nesterov ? nesterov_source(g, m, mu) : m;
  }
  const float mean = block_sum_cw(sum, red) / (float)n;
  float sq = 0.0f;
  for (int64_t i = tid; i < n; i += stride) {
    const float m = buf[i];
    const float s = nesterov ? nesterov_source(muon_grad<GD>(grad, i, inv), m, mu) : m;
    const float d = s - mean;
    sq = fmaf(d, d, sq);
  }
  const float std_all = sqrtf(block_sum_cw(sq, red) / (float)n) + 1e-7f;
  for (int64_t i = tid; i < n; i += stride) {
    const float m = buf[i];
    const float s = nesterov ? nesterov_source(muon_grad<GD>(grad, i, inv), m, mu) : m;
    const float u = s / (n <= 1 ? fabsf(s) + 1e-7f : std_all);
    float x = load1<PD>(p, i);
    if (apply_wd) x = rnd<PD>(x * wd_factor);
    store1<PD>(p, i, rnd<PD>(fmaf(neg_lr, rnd<PD>(u), x)));
  }
}

template <int GD>
void launch_coordwise(float* buf, const void* g, void* p, int32_t p_dtype, int64_t n, float mu, float one_minus_mu,
                      int nesterov, float inv, float wd_factor, int apply_wd, float neg_lr, const apexw_amp_dyn* amp,
                      hipStream_t stream) {
  if (p_dtype == APEXW_F32)
    hipLaunchKernelGGL((muon_coordwise_kernel<GD, APEXW_F32>), dim3(1), dim3(kCwThreads), 0, stream, buf, g, p, n, mu,
                       one_minus_mu, nesterov, inv, wd_factor, apply_wd, neg_lr, amp);
  else if (p_dtype == APEXW_BF16)
    hipLaunchKernelGGL((muon_coordwise_kernel<GD, APEXW_BF16>), dim3(1), dim3(kCwThreads), 0, stream, buf, g, p, n, mu,
                       one_minus_mu, nesterov, inv, wd_factor, apply_wd, neg_lr, amp);
  else
    hipLaunchKernelGGL((muon_coordwise_kernel<GD, APEXW_F16>), dim3(1), dim3(kCwThreads), 0, stream, buf, g, p, n, mu,
                       one_minus_mu, nesterov, inv, wd_factor, apply_wd, neg_lr, amp);
}

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

namespace {

// one grouped launch of the epilogue kind's instantiation (kind without the
// panel bit, which selects kPanel)
template <bool kPanel>
int launch_grouped(const apexw_gemm_problem* probs, const uint32_t* items, const int32_t* offsets, int32_t n_wg,
                   int32_t kind, const apexw_amp_dyn* amp, hipStream_t stream) {
  const dim3 grid(n_wg), block(256);
#define APEXW_GROUPED(C, CT, ADD, NN)                                                                              \
  hipLaunchKernelGGL((gemm_nt_grouped_kernel<C, CT, ADD, NN, kPanel>), grid, block, 0, stream, probs, items, offsets, \
                     amp)
  switch (kind) {
    case APEXW_GEMM_OUT_C: APEXW_GROUPED(true, false, false, false); break;
    case APEXW_GEMM_OUT_C | APEXW_GEMM_ADD: APEXW_GROUPED(true, false, true, false); break;
    case APEXW_GEMM_OUT_CT: APEXW_GROUPED(false, true, false, false); break;
    case APEXW_GEMM_OUT_CT | APEXW_GEMM_ADD: APEXW_GROUPED(false, true, true, false); break;
    case APEXW_GEMM_OUT_C | APEXW_GEMM_OUT_CT: APEXW_GROUPED(true, true, false, false); break;
    case APEXW_GEMM_OUT_C | APEXW_GEMM_OUT_CT | APEXW_GEMM_ADD: APEXW_GROUPED(true, true, true, false); break;
    case APEXW_GEMM_OUT_C | APEXW_GEMM_KIND_NN: APEXW_GROUPED(true, false, false, true); break;
    case APEXW_GEMM_OUT_C | APEXW_GEMM_ADD | APEXW_GEMM_KIND_NN: APEXW_GROUPED(true, false, true, true); break;
    default: return APEXW_ERR_ARG;
  }
#undef APEXW_GROUPED
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

}  // namespace

int apexw_launch_gemm_grouped(const apexw_gemm_problem* probs, const uint32_t* items, const int32_t* offsets,
                              int32_t n_wg, int32_t kind, const apexw_amp_dyn* amp, hipStream_t stream) {
  const int32_t base = kind & ~APEXW_GEMM_KIND_PANEL;
  return (kind & APEXW_GEMM_KIND_PANEL) ? launch_grouped<true>(probs, items, offsets, n_wg, base, amp, stream)
                                        : launch_grouped<false>(probs, items, offsets, n_wg, base, amp, stream);
}

int apexw_muon_partials(int64_t n) { return grid_for(n) < 1024 ? grid_for(n) : 1024; }

template <int GD>
void launch_prepare(float* buf, const void* g, int64_t rows, int64_t cols, float mu, float one_minus_mu, int nesterov,
                    float eps, float inv, uint16_t* x, uint16_t* xt, int64_t ldx, int64_t ldxt, bool panel,
                    float* partial, const apexw_amp_dyn* amp, hipStream_t stream) {
  const int64_t n = rows * cols;
  const int nb = apexw_muon_partials(n);
  if ((((uintptr_t)buf | (uintptr_t)g) & 15u) == 0)
    hipLaunchKernelGGL((muon_momentum_kernel<GD, true>), dim3(nb), dim3(256), 0, stream, buf, g, n, mu, one_minus_mu,
                       nesterov, inv, partial, amp);
  else
    hipLaunchKernelGGL((muon_momentum_kernel<GD, false>), dim3(nb), dim3(256), 0, stream, buf, g, n, mu, one_minus_mu,
                       nesterov, inv, partial, amp);
  dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
  hipLaunchKernelGGL(muon_normalize_kernel<GD>, grid, dim3(256), 0, stream, buf, g, rows, cols, mu, nesterov, inv,
                     partial, nb, eps, (int)(rows > cols), x, xt, ldx, ldxt, panel, amp);
}

int apexw_launch_muon_prepare(float* buf, const void* g, int32_t g_dtype, int64_t rows, int64_t cols, float mu,
                              float one_minus_mu, int32_t nesterov, float eps, float inv, uint16_t* x, uint16_t* xt,
                              int64_t ldx, int64_t ldxt, bool panel, float* partial, const apexw_amp_dyn* amp,
                              hipStream_t stream) {
  if (g_dtype == APEXW_F32)
    launch_prepare<APEXW_F32>(buf, g, rows, cols, mu, one_minus_mu, nesterov, eps, inv, x, xt, ldx, ldxt, panel,
                              partial, amp, stream);
  else if (g_dtype == APEXW_BF16)
    launch_prepare<APEXW_BF16>(buf, g, rows, cols, mu, one_minus_mu, nesterov, eps, inv, x, xt, ldx, ldxt, panel,
                               partial, amp, stream);
  else
    launch_prepare<APEXW_F16>(buf, g, rows, cols, mu, one_minus_mu, nesterov, eps, inv, x, xt, ldx, ldxt, panel,
                              partial, amp, stream);
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

int apexw_launch_muon_apply(void* p, int32_t p_dtype, const uint16_t* u, int64_t rows, int64_t cols, int64_t ldu,
                            bool panel, int32_t u_transposed, float wd_factor, int32_t apply_wd, float neg_lr_eff,
                            const apexw_amp_dyn* amp, hipStream_t stream) {
#define APEXW_APPLY(KERNEL, GRID)                                                                                  \
  hipLaunchKernelGGL(KERNEL, GRID, dim3(256), 0, stream, p, u, rows, cols, ldu, panel, wd_factor, apply_wd,          \
                     neg_lr_eff, amp)
  if (u_transposed) {
    const dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
    if (p_dtype == APEXW_F32) APEXW_APPLY(muon_apply_t_kernel<APEXW_F32>, grid);
    else if (p_dtype == APEXW_BF16) APEXW_APPLY(muon_apply_t_kernel<APEXW_BF16>, grid);
    else APEXW_APPLY(muon_apply_t_kernel<APEXW_F16>, grid);
    return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
  }
  const int64_t n = rows * cols;
  const bool vec = cols % 8 == 0 && ldu % 8 == 0 && (((uintptr_t)p | (uintptr_t)u) & 15u) == 0;
  const dim3 grid(grid_for(vec ? n / 8 : n));
  if (p_dtype == APEXW_F32) {
    if (vec) APEXW_APPLY((muon_apply_kernel<APEXW_F32, true>), grid);
    else APEXW_APPLY((muon_apply_kernel<APEXW_F32, false>), grid);
  } else if (p_dtype == APEXW_BF16) {
    if (vec) APEXW_APPLY((muon_apply_kernel<APEXW_BF16, true>), grid);
    else APEXW_APPLY((muon_apply_kernel<APEXW_BF16, false>), grid);
  } else {
    if (vec) APEXW_APPLY((muon_apply_kernel<APEXW_F16, true>), grid);
    else APEXW_APPLY((muon_apply_kernel<APEXW_F16, false>), grid);
  }
#undef APEXW_APPLY
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}

int apexw_launch_muon_coordwise(float* buf, const void* g, int32_t g_dtype, void* p, int32_t p_dtype, int64_t n,
                                float mu, float one_minus_mu, int32_t nesterov, float inv, float wd_factor,
                                int32_t apply_wd, float neg_lr, const apexw_amp_dyn* amp, hipStream_t stream) {
  if (g_dtype == APEXW_F32)
    launch_coordwise<APEXW_F32>(buf, g, p, p_dtype, n, mu, one_minus_mu, nesterov, inv, wd_factor, apply_wd, neg_lr,
                                amp, stream);
  else if (g_dtype == APEXW_BF16)
    launch_coordwise<APEXW_BF16>(buf, g, p, p_dtype, n, mu, one_minus_mu, nesterov, inv, wd_factor, apply_wd, neg_lr,
                                 amp, stream);
  else
    launch_coordwise<APEXW_F16>(buf, g, p, p_dtype, n, mu, one_minus_mu, nesterov, inv, wd_factor, apply_wd, neg_lr,
                                amp, stream);
  return hipGetLastError() == hipSuccess ? APEXW_OK : APEXW_ERR_LAUNCH;
}
