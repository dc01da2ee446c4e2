// Normalized DotGeneral on gfx950: out[b, m, n] = sum_k lhs[b, m, k] * rhs[b, k, n]
// (rhs[b, n, k] when transposed).  This is the kernel the reference's dot.DotGeneral lowering
// targets (internal/gobackend/dot/dot.go:165-285: [B,M,K] x [B,K,N] "NonTransposed" or
// [B,N,K] "Transposed" layouts, half-precision inputs accumulating into f32).
//
// The tiled kernel stages 64x64 output tiles through LDS, 16-deep in K, each thread owning a
// 4x4 register block; it serves f64, small or unaligned f32 (accumulating in the input type),
// small bf16/f16 (accumulating in f32) and the integer dtypes.  Integers accumulate modulo 2^32
// (2^64 for 64-bit types) in an unsigned register and are stored truncated to the dtype: the low
// bits of a modular sum of modular products are those of Go's wrapping arithmetic in the dtype
// itself (the reference's noSIMD kernels, internal/gobackend/dot/matmul/nosimd.go:66-75), in
// any summation order.  Larger contractions run on the matrix cores: the
// small-tile dot_mm_kernel / dot_mm_lds_kernel below (f32, and half problems too small for
// qdense_gemm.hip's 256x128-tile kernel), or that kernel.

#include <type_traits>

#include "device_common.h"
#include "mxrt_internal.h"

namespace mx {

constexpr int kDotTile = 64;
constexpr int kDotKStep = 16;

template <typename TI, typename TA>
__device__ __forceinline__ TA load_acc(const TI* p, int64_t i, int dt) {
  if constexpr (sizeof(TI) == 2 && std::is_floating_point<TA>::value) {  // bf16 / f16 storage
    const uint16_t h = ((const uint16_t*)p)[i];
    return (TA)(dt == MX_DTYPE_BFLOAT16 ? bf16_to_f32(h) : f16_to_f32(h));
  } else {
    return (TA)p[i];
  }
}

template <typename TI, typename TA, typename TO = TA>
__global__ __launch_bounds__(256) void dot_tiled_kernel(const TI* __restrict__ lhs, const TI* __restrict__ rhs,
                                                        TO* __restrict__ out, int64_t M, int64_t K, int64_t N,
                                                        bool rhs_t, int in_dt) {
  __shared__ TA As[kDotKStep][kDotTile + 1];
  __shared__ TA Bs[kDotKStep][kDotTile + 1];
  const int64_t b = blockIdx.z;
  const int64_t m0 = (int64_t)blockIdx.y * kDotTile, n0 = (int64_t)blockIdx.x * kDotTile;
  const TI* L = lhs + b * M * K;
  const TI* R = rhs + b * K * N;
  const int tid = threadIdx.x;
  const int ty = tid / 16, tx = tid % 16;
  TA acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (TA)0;
  for (int64_t k0 = 0; k0 < K; k0 += kDotKStep) {
    // 64x16 tiles = 1024 elements, 4 per thread.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = tid + e * 256;
      {  // lhs: As[kk][mm] = L[m0+mm, k0+kk]
        const int kk = idx % kDotKStep, mm = idx / kDotKStep;
        const int64_t m = m0 + mm, k = k0 + kk;
        As[kk][mm] = (m < M && k < K) ? load_acc<TI, TA>(L, m * K + k, in_dt) : (TA)0;
      }
      if (!rhs_t) {  // Bs[kk][nn] = R[k0+kk, n0+nn]
        const int nn = idx % kDotTile, kk = idx / kDotTile;
        const int64_t n = n0 + nn, k = k0 + kk;
        Bs[kk][nn] = (n < N && k < K) ? load_acc<TI, TA>(R, k * N + n, in_dt) : (TA)0;
      } else {  // Bs[kk][nn] = R[n0+nn, k0+kk]
        const int kk = idx % kDotKStep, nn = idx / kDotKStep;
        const int64_t n = n0 + nn, k = k0 + kk;
        Bs[kk][nn] = (n < N && k < K) ? load_acc<TI, TA>(R, n * K + k, in_dt) : (TA)0;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kDotKStep; ++kk) {
      TA a[4], bb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bb[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * bb[j];
    }
    __syncthreads();
  }
  TO* O = out + b * M * N;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + ty * 4 + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n < N) O[m * N + n] = (TO)acc[i][j];
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Small-tile DotGeneral on the matrix cores, for f32 inputs (v_mfma_f32_16x16x4_f32: fp32
// products and sums, twice the dense rate the VALU reaches without packed fp32) and for half
// inputs whose problem is too small to fill the chip with qdense_gemm.hip's 256x128 tiles
// (v_mfma_f32_16x16x32_bf16 / _f16: exact products, f32 sums).  Either way the result differs
// from a sequential f32 sum only in summation order.
//
// A workgroup (4 waves) owns a (16*TM*WM) x (16*TN*WN) output tile; WM x WN waves split the
// tile and the remaining KS = 4 / (WM*WN) waves split K (wave w takes K steps w, w+KS, ...),
// summed through LDS in wave order at the end (deterministic).  Operands come straight from
// global memory into registers, one step ahead: a wave's K step is 32 deep, lane group g
// (lane / 16) holding k = 8g .. 8g+7 of row (lane % 16) of each 16-row A tile and the same k
// of column (lane % 16) of each 16-column B tile.  In f32 MFMA t contracts k = {8g + t}; in
// half one MFMA contracts all 32 (its lane layout is exactly this one).  Every lane group
// reads a contiguous run of its row.  Rows, columns and k beyond the problem load clamped
// (in-bounds) addresses and are zeroed by a select when the step is used, so the loads are
// not waited on where they issue.  f32 needs K % 4 == 0, half K % 8 == 0.
// ---------------------------------------------------------------------------------------------
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_v;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_v;
constexpr int kMmStep = 32;
enum DotKind { kDkF32 = 0, kDkBf16 = 1, kDkF16 = 2 };

// Raw operands of one K step: 8 f32 or 8 halves (4 words) per tile per lane.
template <int KIND, bool BT, int TM, int TN>
__device__ __forceinline__ void dot_mm_load(const void* const (&ap)[TM], const void* const (&bp)[TN], int kb, int g,
                                            int K, int N, uint32_t (&ra)[TM][8], uint32_t (&rb)[TN][8]) {
  const int k0 = kb + 8 * g;
  if constexpr (KIND == kDkF32) {
    const int c0 = min(k0, K - 4), c1 = min(k0 + 4, K - 4);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const u32x4_t lo = *((const u32x4_t*)((const float*)ap[i] + c0)), hi = *((const u32x4_t*)((const float*)ap[i] + c1));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ra[i][e] = lo[e];
        ra[i][4 + e] = hi[e];
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (BT) {
        const u32x4_t lo = *((const u32x4_t*)((const float*)bp[j] + c0)), hi = *((const u32x4_t*)((const float*)bp[j] + c1));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          rb[j][e] = lo[e];
          rb[j][4 + e] = hi[e];
        }
      } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) rb[j][t] = ((const uint32_t*)bp[j])[(int64_t)min(k0 + t, K - 1) * N];
      }
    }
  } else {
    const int c0 = min(k0, K - 8);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const u32x4_t v = *((const u32x4_t*)((const uint16_t*)ap[i] + c0));
#pragma unroll
      for (int e = 0; e < 4; ++e) ra[i][e] = v[e];
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (BT) {
        const u32x4_t v = *((const u32x4_t*)((const uint16_t*)bp[j] + c0));
#pragma unroll
        for (int e = 0; e < 4; ++e) rb[j][e] = v[e];
      } else {
        const uint16_t* q = (const uint16_t*)bp[j];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          rb[j][e] = (uint32_t)q[(int64_t)min(k0 + 2 * e, K - 1) * N] |
                     ((uint32_t)q[(int64_t)min(k0 + 2 * e + 1, K - 1) * N] << 16);
      }
    }
  }
}

template <int KIND, int TM, int TN>
__device__ __forceinline__ void dot_mm_mask(int kb, int g, int K, const uint32_t (&ra)[TM][8], const uint32_t (&rb)[TN][8],
                                            uint32_t (&a)[TM][8], uint32_t (&bv)[TN][8]) {
  const int k0 = kb + 8 * g;
  constexpr int W = KIND == kDkF32 ? 8 : 4;  // words per tile; a half word is valid as a whole
#pragma unroll
  for (int t = 0; t < W; ++t) {
    const bool v = KIND == kDkF32 ? k0 + t < K : k0 < K;
#pragma unroll
    for (int i = 0; i < TM; ++i) a[i][t] = v ? ra[i][t] : 0u;
#pragma unroll
    for (int j = 0; j < TN; ++j) bv[j][t] = v ? rb[j][t] : 0u;
  }
}

template <int KIND>
__device__ __forceinline__ f32x4_t dot_mm_step(const uint32_t (&a)[8], const uint32_t (&b)[8], f32x4_t c) {
  if constexpr (KIND == kDkF32) {
#pragma unroll
    for (int t = 0; t < 8; ++t) c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[t]), __uint_as_float(b[t]), c, 0, 0, 0);
    return c;
  } else {
    const u32x4_t av{a[0], a[1], a[2], a[3]}, bw{b[0], b[1], b[2], b[3]};
    if constexpr (KIND == kDkBf16)
      return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, av), __builtin_bit_cast(bf16x8_v, bw), c, 0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_v, av), __builtin_bit_cast(f16x8_v, bw), c, 0, 0, 0);
  }
}

// out_half: 0 stores f32; otherwise the output is the input's half dtype, rounded once to
// nearest even.
template <int KIND, bool BT, int WM, int WN, int TM, int TN>
__global__ __launch_bounds__(256) void dot_mm_kernel(const void* __restrict__ lhs, const void* __restrict__ rhs,
                                                     void* __restrict__ out, int M, int K, int N, int out_half) {
  constexpr int KS = 4 / (WM * WN);
  constexpr int ES = KIND == kDkF32 ? 4 : 2;  // input element bytes
  static_assert(KS * WM * WN == 4, "4 waves");
  __shared__ f32x4_t red[KS > 1 ? (KS - 1) * WM * WN * TM * TN * 64 : 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wk = wave % KS, wmn = wave / KS, wm = wmn / WN, wn = wmn % WN;
  const int r = lane & 15, g = lane >> 4;
  const int64_t bz = blockIdx.z;
  const int m0 = blockIdx.y * (16 * TM * WM) + wm * 16 * TM;
  const int n0 = blockIdx.x * (16 * TN * WN) + wn * 16 * TN;
  const char* L = (const char*)lhs + bz * M * K * ES;
  const char* R = (const char*)rhs + bz * K * N * ES;
  const void* ap[TM];
  const void* bp[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) ap[i] = L + (int64_t)min(m0 + 16 * i + r, M - 1) * K * ES;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = min(n0 + 16 * j + r, N - 1);
    bp[j] = BT ? R + (int64_t)n * K * ES : R + (int64_t)n * ES;
  }
  f32x4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int steps = (K + kMmStep - 1) / kMmStep;
  uint32_t ra[TM][8], rb[TN][8];
  dot_mm_load<KIND, BT, TM, TN>(ap, bp, wk * kMmStep, g, K, N, ra, rb);
  for (int s = wk; s < steps; s += KS) {
    uint32_t a[TM][8], bv[TN][8];
    dot_mm_mask<KIND, TM, TN>(s * kMmStep, g, K, ra, rb, a, bv);
    // Next step's operands (the last step reloads itself: in bounds, unused), issued ahead of
    // this step's products.
    dot_mm_load<KIND, BT, TM, TN>(ap, bp, min(s + KS, steps - 1) * kMmStep, g, K, N, ra, rb);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = dot_mm_step<KIND>(a[i], bv[j], acc[i][j]);
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (KS > 1) {
    if (wk > 0) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) red[(((wk - 1) * WM * WN + wmn) * TM * TN + i * TN + j) * 64 + lane] = acc[i][j];
    }
    __syncthreads();
    if (wk > 0) return;
#pragma unroll
    for (int w = 1; w < KS; ++w)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] += red[(((w - 1) * WM * WN + wmn) * TM * TN + i * TN + j) * 64 + lane];
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + 16 * j + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 16 * i + 4 * g + e;
        if (m >= M || n >= N) continue;
        const int64_t o = bz * M * N + (int64_t)m * N + n;
        const float v = acc[i][j][e];
        if (!out_half)
          ((float*)out)[o] = v;
        else
          ((uint16_t*)out)[o] = KIND == kDkBf16 ? f32_to_bf16(v) : f32_to_f16(v);
      }
    }
}

// LDS-staged variant for a transposed right-hand side ([N, K]; the normalized layout of every
// projection in the reference's model benchmarks): a 64x64 tile per workgroup, its 4 waves 2x2
// over 32x32, K steps of 32 staged through two LDS buffers.  All 256 threads load A and B
// rows together, 8 (f32) or 4 (half) lanes per contiguous row segment, so each element is
// loaded once per workgroup and each load instruction touches whole row segments; the waves
// then read their fragments in the MFMA layout above (lane group g: k = 8g .. 8g+7) from rows
// padded by 16 bytes, which keeps each 16-lane read on distinct banks.  With KS2 = 2 the
// workgroup has 8 waves: each half (256 threads) loads and multiplies alternate K steps, and
// the halves' sums are added through LDS at the end (two waves per SIMD when the grid has
// fewer tiles than CUs).
template <int KIND, int KS2>
__global__ __launch_bounds__(256 * KS2) void dot_mm_lds_kernel(const void* __restrict__ lhs, const void* __restrict__ rhs,
                                                               void* __restrict__ out, int M, int K, int N, int out_half) {
  constexpr int ES = KIND == kDkF32 ? 4 : 2;
  constexpr int RB = kMmStep * ES, RS = RB + 16;  // row bytes per step; padded LDS row stride
  constexpr int LPR = RB / 16;                     // 16-byte chunks per row segment
  constexpr int PASSES = 64 * LPR / 256;           // 16-byte loads per thread per operand
  __shared__ __attribute__((aligned(16))) char sm[2][KS2][2][64 * RS];
  const int part = threadIdx.x >> 8, tid = threadIdx.x & 255, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1, r = lane & 15, g = lane >> 4;
  const int64_t bz = blockIdx.z;
  const int mt = blockIdx.y * 64, nt = blockIdx.x * 64;
  const char* L = (const char*)lhs + bz * M * K * ES;
  const char* R = (const char*)rhs + bz * K * N * ES;
  const int c = tid % LPR, row0 = tid / LPR;  // this thread's chunk and first row
  const char* ga[PASSES];
  const char* gb[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int row = row0 + p * (256 / LPR);
    ga[p] = L + (int64_t)min(mt + row, M - 1) * K * ES;
    gb[p] = R + (int64_t)min(nt + row, N - 1) * K * ES;
  }
  // Global loads run two K steps ahead of the products, in two register sets X and Y (even and
  // odd steps) with the loop unrolled by two so both stay static.  Steps past the end load
  // clamped addresses and store zeros (lstore's K mask), so an odd last pair adds nothing.
  const int steps = (K + kMmStep - 1) / kMmStep;
  u32x4_t xa[PASSES], xb[PASSES], ya[PASSES], yb[PASSES];
  auto gload = [&](int s, u32x4_t (&va)[PASSES], u32x4_t (&vb)[PASSES]) {
    // A chunk holds 4 (f32) or 8 (half) k: wholly inside K or wholly past it (K % 4 / K % 8);
    // one past it loads the row's last chunk instead (in bounds) and is zeroed by lstore.
    const int64_t off = (int64_t)min((s * KS2 + part) * kMmStep + c * (16 / ES), K - 16 / ES) * ES;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      va[p] = *(const u32x4_t*)(ga[p] + off);
      vb[p] = *(const u32x4_t*)(gb[p] + off);
    }
  };
  auto lstore = [&](int s, int buf, const u32x4_t (&va)[PASSES], const u32x4_t (&vb)[PASSES]) {
    const bool v = (s * KS2 + part) * kMmStep + c * (16 / ES) < K;
    const u32x4_t z{0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = row0 + p * (256 / LPR);
      *(u32x4_t*)(&sm[buf][part][0][row * RS + c * 16]) = v ? va[p] : z;
      *(u32x4_t*)(&sm[buf][part][1][row * RS + c * 16]) = v ? vb[p] : z;
    }
  };
  f32x4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int buf) {
    uint32_t a[2][8], bv[2][8];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const char* pa = &sm[buf][part][0][(wm * 32 + 16 * i + r) * RS + g * 8 * ES];
      const char* pb = &sm[buf][part][1][(wn * 32 + 16 * i + r) * RS + g * 8 * ES];
#pragma unroll
      for (int h = 0; h < 8 * ES / 16; ++h) {
        const u32x4_t x = *(const u32x4_t*)(pa + 16 * h), y = *(const u32x4_t*)(pb + 16 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a[i][4 * h + e] = x[e];
          bv[i][4 * h + e] = y[e];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = dot_mm_step<KIND>(a[i], bv[j], acc[i][j]);
  };
  const int nq = (steps + KS2 - 1) / KS2;  // step groups (one step per half)
  // The scheduling barriers keep each set's loads where they are issued, so a store waits only
  // for the older set.
  gload(0, xa, xb);
  __builtin_amdgcn_sched_barrier(0);
  gload(1, ya, yb);
  __builtin_amdgcn_sched_barrier(0);
  lstore(0, 0, xa, xb);
  __syncthreads();
  for (int s = 0; s < nq; s += 2) {
    gload(s + 2, xa, xb);
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    lstore(s + 1, 1, ya, yb);
    __syncthreads();
    gload(s + 3, ya, yb);
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    lstore(s + 2, 0, xa, xb);
    __syncthreads();
  }
  if constexpr (KS2 > 1) {
    // The loop ended on a barrier: the LDS buffers are free.  Half 1 hands its sums to half 0.
    f32x4_t* red = (f32x4_t*)&sm[0][0][0][0];
    if (part == 1) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) red[(wave * 4 + i * 2 + j) * 64 + lane] = acc[i][j];
    }
    __syncthreads();
    if (part == 1) return;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] += red[(wave * 4 + i * 2 + j) * 64 + lane];
  }
  const int m0 = mt + wm * 32, n0 = nt + wn * 32;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + 16 * j + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 16 * i + 4 * g + e;
        if (m >= M || n >= N) continue;
        const int64_t o = bz * M * N + (int64_t)m * N + n;
        const float v = acc[i][j][e];
        if (!out_half)
          ((float*)out)[o] = v;
        else
          ((uint16_t*)out)[o] = KIND == kDkBf16 ? f32_to_bf16(v) : f32_to_f16(v);
      }
    }
}

static int dot_kind(int dt) {
  return dt == MX_DTYPE_FLOAT32 ? kDkF32 : dt == MX_DTYPE_BFLOAT16 ? kDkBf16 : dt == MX_DTYPE_FLOAT16 ? kDkF16 : -1;
}

// Large enough contractions (>= 2^20 multiply-adds) with 16-byte aligned operands: f32 with
// K % 4 == 0 (small ones keep the tiled kernel's sequential sums), half with K % 8 == 0 and f32
// or half output.
static bool dot_mm_fits(const DotDesc& d) {
  auto aligned = [](const void* p, size_t al) { return ((uintptr_t)p % al) == 0; };
  const int kind = dot_kind(d.in_dt);
  if (kind < 0 || !(d.out_dt == MX_DTYPE_FLOAT32 || d.out_dt == d.in_dt)) return false;
  const int kal = kind == kDkF32 ? 4 : 8;
  return d.K >= kal && d.K % kal == 0 && d.B * d.M * d.N * d.K >= ((int64_t)1 << 20) && d.B <= 65535 &&
         d.M < (1 << 24) && d.N < (1 << 24) && d.K < (1 << 24) && aligned(d.lhs, 16) && aligned(d.rhs, 16);
}

template <int KIND, bool BT, int WM, int WN, int TM, int TN>
static int dot_mm_launch(mx_backend* b, const DotDesc& d, const char* name) {
  constexpr int BM = 16 * TM * WM, BN = 16 * TN * WN;
  const dim3 grid((unsigned)((d.N + BN - 1) / BN), (unsigned)((d.M + BM - 1) / BM), (unsigned)d.B);
  if (grid.y > 65535u) return set_error(MX_ERR_INVALID, "DotGeneral: M too large");
  hipStream_t st = b->stream;
  const int out_half = d.out_dt == MX_DTYPE_FLOAT32 ? 0 : 1;
  return launch(b, name, [&] {
    dispatch(dot_mm_kernel<KIND, BT, WM, WN, TM, TN>, grid, 256, 0, st, d.lhs, d.rhs, d.out, (int)d.M, (int)d.K, (int)d.N,
             out_half);
  });
}

template <int KIND>
static int dot_mm_lds_launch(mx_backend* b, const DotDesc& d, const char* name) {
  const dim3 grid((unsigned)((d.N + 63) / 64), (unsigned)((d.M + 63) / 64), (unsigned)d.B);
  if (grid.y > 65535u) return set_error(MX_ERR_INVALID, "DotGeneral: M too large");
  hipStream_t st = b->stream;
  const int out_half = d.out_dt == MX_DTYPE_FLOAT32 ? 0 : 1;
  // Fewer tiles than CUs and several K steps: 8 waves splitting K.
  const bool split = (int64_t)grid.x * grid.y * grid.z < 256 && d.K >= 8 * kMmStep;
  return launch(b, name, [&] {
    if (split)
      dispatch(dot_mm_lds_kernel<KIND, 2>, grid, 512, 0, st, d.lhs, d.rhs, d.out, (int)d.M, (int)d.K, (int)d.N, out_half);
    else
      dispatch(dot_mm_lds_kernel<KIND, 1>, grid, 256, 0, st, d.lhs, d.rhs, d.out, (int)d.M, (int)d.K, (int)d.N, out_half);
  });
}

// Tile choice: a transposed right-hand side with >= 128 64x64 tiles stages them through LDS;
// otherwise the largest register tile that still gives >= 512 workgroups, K-split waves only
// when each has several K steps.
template <int KIND, bool BT>
static int dot_mm_select(mx_backend* b, const DotDesc& d, const char* name) {
  auto wgs = [&](int bm, int bn) { return d.B * ((d.M + bm - 1) / bm) * ((d.N + bn - 1) / bn); };
  if constexpr (BT) {
    if (wgs(64, 64) >= 128) return dot_mm_lds_launch<KIND>(b, d, name);
  }
  const int64_t steps = (d.K + kMmStep - 1) / kMmStep;
  if (wgs(64, 64) >= 512) return dot_mm_launch<KIND, BT, 2, 2, 2, 2>(b, d, name);
  if (steps < 8) return dot_mm_launch<KIND, BT, 2, 2, 1, 1>(b, d, name);
  if (wgs(32, 32) >= 512) return dot_mm_launch<KIND, BT, 1, 1, 2, 2>(b, d, name);
  return dot_mm_launch<KIND, BT, 1, 1, 1, 2>(b, d, name);
}

static int dot_mm_run(mx_backend* b, const DotDesc& d) {
  const bool bt = d.rhs_transposed;
  switch (dot_kind(d.in_dt)) {
    case kDkF32:
      return bt ? dot_mm_select<kDkF32, true>(b, d, "dot_mfma_f32") : dot_mm_select<kDkF32, false>(b, d, "dot_mfma_f32");
    case kDkBf16:
      return bt ? dot_mm_select<kDkBf16, true>(b, d, "dot_mfma_bf16_tile")
                : dot_mm_select<kDkBf16, false>(b, d, "dot_mfma_bf16_tile");
    default:
      return bt ? dot_mm_select<kDkF16, true>(b, d, "dot_mfma_f16_tile")
                : dot_mm_select<kDkF16, false>(b, d, "dot_mfma_f16_tile");
  }
}

// qdense_gemm.hip's 256x128-tile kernel takes half contractions with M >= 256 that give it
// >= 64 workgroups (measured: at 96 it beats the small tiles 12 us to 22 us; at 24 or fewer,
// or batched with M = 128 / 192, the small tiles win); others go to the small-tile kernels.
static bool dot_big_tiles(const DotDesc& d) {
  return dot_mfma_fits(d) && d.M >= 256 && d.B * ((d.M + 255) / 256) * ((d.N + 127) / 128) >= 64;
}

int dot_run(mx_backend* b, const DotDesc& d) {
  MX_TRY(check_device(b));
  if (d.B == 0 || d.M == 0 || d.N == 0) return MX_OK;
  if (d.K == 0) {
    const size_t bytes = (size_t)d.B * d.M * d.N * (dtype_bits(d.out_dt) / 8);
    MX_CHECK_HIP(hipMemsetAsync(d.out, 0, bytes, b->stream));
    return MX_OK;
  }
  if (dot_big_tiles(d))
    return dot_mfma_run(b, d, d.in_dt == MX_DTYPE_BFLOAT16 ? "dot_mfma_bf16" : "dot_mfma_f16");
  if (dot_mm_fits(d)) return dot_mm_run(b, d);
  if (dot_mfma_fits(d))
    return dot_mfma_run(b, d, d.in_dt == MX_DTYPE_BFLOAT16 ? "dot_mfma_bf16" : "dot_mfma_f16");
  if (dtype_is_half(d.in_dt) && d.out_dt != MX_DTYPE_FLOAT32) {
    // Half output folded in by the graph compiler, on a path that sums into f32 memory: the f32
    // result goes to a temporary, then ConvertDType's own kernel rounds it (the same arithmetic).
    void* tmp = nullptr;
    const int64_t n = d.B * d.M * d.N;
    MX_TRY(dev_alloc(b, (size_t)n * sizeof(float), &tmp));
    DotDesc d2 = d;
    d2.out = tmp;
    d2.out_dt = MX_DTYPE_FLOAT32;
    int rc = dot_run(b, d2);
    if (rc == MX_OK) rc = ew_convert(b, tmp, MX_DTYPE_FLOAT32, d.out, d.out_dt, n);
    dev_free(b, tmp);  // stream-ordered pool: later users run after these kernels
    return rc;
  }
  if (d.B > 65535) return set_error(MX_ERR_INVALID, "DotGeneral: batch size %lld too large", (long long)d.B);
  dim3 grid((unsigned)((d.N + kDotTile - 1) / kDotTile), (unsigned)((d.M + kDotTile - 1) / kDotTile), (unsigned)d.B);
  if (grid.y > 65535u) return set_error(MX_ERR_INVALID, "DotGeneral: M too large");
  hipStream_t st = b->stream;
  switch (d.in_dt) {
    case MX_DTYPE_FLOAT32:
      return launch(b, "dot_tiled_f32", [&] {
        dispatch(dot_tiled_kernel<float, float>, grid, 256, 0, st, (const float*)d.lhs, (const float*)d.rhs, (float*)d.out, d.M,
                                                              d.K, d.N, d.rhs_transposed, d.in_dt);
      });
    case MX_DTYPE_FLOAT64:
      return launch(b, "dot_tiled_f64", [&] {
        dispatch(dot_tiled_kernel<double, double>, grid, 256, 0, st, (const double*)d.lhs, (const double*)d.rhs,
                                                                (double*)d.out, d.M, d.K, d.N, d.rhs_transposed, d.in_dt);
      });
    case MX_DTYPE_BFLOAT16:
    case MX_DTYPE_FLOAT16:
      return launch(b, d.in_dt == MX_DTYPE_BFLOAT16 ? "dot_tiled_bf16" : "dot_tiled_f16", [&] {
        dispatch(dot_tiled_kernel<uint16_t, float>, grid, 256, 0, st, (const uint16_t*)d.lhs, (const uint16_t*)d.rhs,
                                                                 (float*)d.out, d.M, d.K, d.N, d.rhs_transposed, d.in_dt);
      });
    default:
      break;
  }
  // Integers: the output dtype is the input's (the graph converts to the accumulator dtype first).
  auto int_dot = [&](auto ti, auto ta, const char* name) {
    using TI = decltype(ti);
    using TA = decltype(ta);
    return launch(b, name, [&] {
      dispatch(dot_tiled_kernel<TI, TA, TI>, grid, 256, 0, st, (const TI*)d.lhs, (const TI*)d.rhs, (TI*)d.out, d.M, d.K,
               d.N, d.rhs_transposed, d.in_dt);
    });
  };
  if (d.out_dt != d.in_dt)
    return set_error(MX_ERR_NOT_IMPLEMENTED, "DotGeneral: %s inputs with %s output", dtype_name(d.in_dt),
                     dtype_name(d.out_dt));
  switch (d.in_dt) {
    case MX_DTYPE_INT8: return int_dot(int8_t{}, uint32_t{}, "dot_tiled_i8");
    case MX_DTYPE_UINT8: return int_dot(uint8_t{}, uint32_t{}, "dot_tiled_u8");
    case MX_DTYPE_INT16: return int_dot(int16_t{}, uint32_t{}, "dot_tiled_i16");
    case MX_DTYPE_UINT16: return int_dot(uint16_t{}, uint32_t{}, "dot_tiled_u16");
    case MX_DTYPE_INT32: return int_dot(int32_t{}, uint32_t{}, "dot_tiled_i32");
    case MX_DTYPE_UINT32: return int_dot(uint32_t{}, uint32_t{}, "dot_tiled_u32");
    case MX_DTYPE_INT64: return int_dot(int64_t{}, uint64_t{}, "dot_tiled_i64");
    case MX_DTYPE_UINT64: return int_dot(uint64_t{}, uint64_t{}, "dot_tiled_u64");
    default:
      return set_error(MX_ERR_NOT_IMPLEMENTED, "DotGeneral: dtype %s not implemented", dtype_name(d.in_dt));
  }
}

}  // namespace mx
