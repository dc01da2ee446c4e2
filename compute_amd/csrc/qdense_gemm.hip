// Prefill FusedQuantizedDense on gfx950: a bf16 MFMA GEMM with the Int8 / Uint8 / Int4 / Uint4
// weights dequantised on the fly, for M > 16 rows of bf16 activations and one scale per output
// column or per group of G rows (G a multiple of 64) and output column.
//
// Reference semantics: quantizedDenseLinearInt (internal/gobackend/fusedops/quantizeddense.go:
// 616-650, the 4-bit unpack at :383-390) then the activation epilogue (fusedops/dense.go:176-205).
// The reference's terms (x*w)*s factor per scale group:
//   y[m,n] = act(bias[n] + sum_g s[g,n] * sum_{k in g} x[m,k]*w[k,n]),
// with one group for per-channel scales; every product x*w is exact in f32 (bf16 x, |w| < 256),
// so only the summation order differs from the reference.  With groups, the MFMAs accumulate
// into a second set of registers that is folded into the total with the group's scales
// (acc += accg * s[g]): with bf16 scales after every 64-row block (its first MFMAs start from
// zero, so nothing is cleared), with f32 scales at the group's last block.
//
// Tiling.  A workgroup (8 waves, two per SIMD) computes a 256 x 128 output tile; wave w owns
// rows [64 wr, 64 wr + 64) x columns [64 wc, 64 wc + 64) with wr = w % 4, wc = w / 4.  K advances
// in blocks of 64 (two 32-row steps of v_mfma_f32_16x16x32_bf16).  LDS holds
//   - x, four buffers (three with f32 group scales): [256 rows][64 k] bf16; 16-byte k-chunks XOR-swizzled within each row by
//     (row >> 1) & 7 so that an MFMA operand read (16 rows) hits distinct banks;
//   - Bt, two buffers: [128 columns][64 k] bf16, the weights converted exactly to bf16 (|w| < 256
//     has at most 8 significant bits) and transposed.  Column c is stored in row p = c ^ ((c >> 2)
//     & 1) and its 16-byte k-chunks are XOR-swizzled by (p >> 3) & 7: the 16 lanes of a B-operand
//     read (columns 4 apart) then cover both halves of the banks and 8 distinct chunks in each.
// x moves straight from memory into its LDS buffer (global_load_lds_dwordx4, 1 KB = 8 rows per
// wave instruction, the swizzle applied by choosing each lane's source chunk) three blocks ahead of
// its use (two with f32 group scales), and takes no registers, VALU or LDS-write instructions; that leaves room for the
// grouped kernels' second accumulator set beside a full 256 x 128 tile.  The weights travel
// through registers (loads of block kb + PF issued during block kb, each thread 4 rows x 4
// columns: 4 bytes of int8, 2 of 4-bit or 8 of a half type per row; 32 threads per row segment),
// are converted and written transposed into the Bt buffer of block kb + 1 during block kb.
// One barrier per block publishes the next block (each wave first waits for its own x loads of
// it: the loads are issued in a fixed order, so a count of outstanding loads names them) and
// retires the reads of the current buffers; it sits between the block's two steps, so that the
// next block's step-0 operand reads travel under step 1's MFMAs.  sched_group_barrier interleaves
// the memory instructions one per MFMA: issuing a global load or an LDS access can stall the
// wave, and a stall that overlaps an MFMA in flight costs nothing.  Loads past the last block
// re-read it (clamped index), which keeps the count of loads per block fixed.
// Lane (cg = lane % 16, kq = lane / 16) ends with rows 4*kq + r of each 16-row block and the 4
// consecutive columns 4*cg .. 4*cg + 3 of its wave's 64; the epilogue applies scale, bias and
// activation and writes 8-byte bf16 runs.
// Tile order: every XCD (workgroups are dispatched round-robin over the 8) takes a 2 x 16 block
// of tiles, so its L2 serves the x rows and w columns they share.
#include <algorithm>
#include <type_traits>

#include "device_common.h"
#include "mxrt_internal.h"

namespace mx {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_v __attribute__((ext_vector_type(2)));
constexpr int kBM = 256, kBN = 128, kBK = 64, kWaves = 8, kThreads = 64 * kWaves;
constexpr int kABytes = kBM * kBK * 2;   // 32 KB per x buffer
constexpr int kBtBytes = kBN * kBK * 2;  // 16 KB per Bt buffer
// x buffers: a block's rows are requested kXBufs - 1 blocks ahead of its use.  Four (160 KB of
// LDS with the two Bt buffers) except for f32 group scales, whose run-time group branch leaves no
// registers for the longer wait (three: 128 KB).  Q1 360 -> 351 us, Q2 360 -> 346 us, D1 98 -> 95 us
// per call with four; C4 unchanged.
template <int BK, bool GRP, bool FB>
constexpr int kXBufs = (GRP && !FB) ? 3 : 4;
constexpr int kXDma = kABytes / (kWaves * 1024);     // 1 KB direct-to-LDS loads per wave per block
constexpr int kWLoads = 4;                           // w loads (one per row) per thread per block
constexpr int kPf = 4;                               // w blocks loaded ahead into registers
constexpr int kUnroll = 4;                           // multiple of kPf and of the 2 Bt buffers
constexpr int64_t kSplitPlanCUs = 256;               // CUs the split tail is planned for (MI355X)
static_assert(kXDma * kWaves * 1024 == kABytes, "x load split");
static_assert(kBK * kBN == 16 * kThreads, "conversion: 16 weights per thread");

// B operand kinds: the quantized weights [K, N] (int8 / uint8, converted to bf16), or a
// DotGeneral right-hand side in bf16 / f16, [K, N] (transposed on the way into LDS) or [N, K].
enum GemmB { kBI8 = 0, kBU8, kBI4, kBU4, kBBf16KN, kBF16KN, kBBf16NK, kBF16NK };
template <int BK> constexpr bool kDotB = BK >= kBBf16KN;
template <int BK> constexpr bool k4B = BK == kBI4 || BK == kBU4;
template <int BK> constexpr bool kF16B = BK == kBF16KN || BK == kBF16NK;
template <int BK> constexpr bool kNKB = BK == kBBf16NK || BK == kBF16NK;

struct GemmArgs {
  const uint16_t* x;  // [batch][M, K] bf16 (f16 with an f16 B)
  const uint8_t* w;   // [K, N] int8 / uint8, or [batch][K, N] / [batch][N, K] half
  const void* scale;  // [N] (quantized)
  const void* bias;   // [N] or null (quantized)
  void* out;          // [M, N] bf16 (quantized) or [batch][M, N] f32 / bf16 / f16 (DotGeneral)
  int M, K, N, s_dt, b_dt, act, tiles_n, grouped, tiles, out_dt;
  int gpb;            // blocks of 64 K rows per scale group (grouped scales; scale is [K/G, N])
  // Split tail (quantized kernels): work items [0, split_from) are whole tiles; the last
  // (gridDim.x - split_from) / 2 tiles are computed as two halves of K each, by consecutive
  // workgroups, which exchange f32 partial tiles through `part` (scratch) and count arrivals in
  // `ctr` (zero between launches); the second to arrive adds the halves (half 0 + half 1) and
  // stores the tile.  split_from == gridDim.x: no split.
  int split_from;
  float* part;        // [tail tiles][2 halves][16][512 threads][4] f32
  uint32_t* ctr;      // [tail tiles]
};

template <int BK>
__device__ __forceinline__ f32x4_t mfma(const u32x4_v& a, const u32x4_v& b, f32x4_t c) {
  if constexpr (kF16B<BK>)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

// Workgroup barrier ordering LDS only: waits for this wave's LDS accesses, not for its global
// loads in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// LDS byte address of a shared-memory pointer.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// Direct memory-to-LDS load of 16 bytes per lane from base + voff (base wave-uniform, voff the
// lane's byte offset): lane l's bytes land at LDS address lds_base + 16 * l (lds_base
// wave-uniform, held in M0 for the instruction, which is saved and restored around it).  Issued as assembly: the compiler neither waits for it nor knows that it
// writes LDS, so the kernel waits for it itself (wait_vm) before the barrier that publishes the
// block, and the "memory" clobber keeps every compiler memory access in program order around it.
// The memory counter completes loads in issue order, so the compiler's own waits for its later
// or earlier loads stay correct (they only cover these as well).
__device__ __forceinline__ void lds_dma_b128(const void* base, uint32_t voff, uint32_t lds_base) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(lds_base), "s"(base)
      : "memory");
}

// Waits until at most N of this wave's memory loads are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N == 6 || N == 8 || N == 12 || N == 16, "counts used by the kernel");
  if constexpr (N == 6)
    asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else if constexpr (N == 8)
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else if constexpr (N == 12)
    asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
}

typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;

// act(v * s + b) for two columns, rounded to a bf16 pair by the hardware conversion
// (v_cvt_pk_bf16_f32: round to nearest even, the same bits as f32_to_bf16 for every non-NaN
// value), for a compile-time activation.
template <int ACT>
__device__ __forceinline__ uint32_t scaled_act_bf16x2(float v0, float s0, float b0, float v1, float s1, float b1) {
  const f32x2_t y = {act_fast(v0 * s0 + b0, ACT), act_fast(v1 * s1 + b1, ACT)};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(y, bf16x2_t));
}

// Epilogue of one lane: scale, bias, activation, bf16, 8-byte stores of 4 consecutive columns
// per row.  The activation is a template parameter so that each variant is straight-line code
// (no calls, which would save and restore the live accumulators around every one).
template <int ACT>
__device__ __forceinline__ void store_tile(const f32x4_t (&acc)[4][4], const float (&sc)[4], const float (&bi)[4],
                                           uint16_t* out, int row0, int M, size_t N, int ncol) {
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = row0 + 16 * rb + r;
      if (row < M) {
        uint32_t o[2];
#pragma unroll
        for (int c = 0; c < 4; c += 2)
          o[c / 2] = scaled_act_bf16x2<ACT>(acc[rb][c][r], sc[c], bi[c], acc[rb][c + 1][r], sc[c + 1], bi[c + 1]);
        *(uint2*)(out + (size_t)row * N + ncol) = make_uint2(o[0], o[1]);
      }
    }
  }
}

// FB (scale groups with bf16 scales): every block's MFMA sums start from zero (C operand 0) and
// are folded into the total with the scales of the block's group at the block's end, so there is
// no clearing and no per-block branch (a group of G = 64 j rows is folded j times, once per
// block).  Otherwise groups are counted at run time and the sums cleared after each fold.
// H (with FB): scale groups of 32 rows, two per 64-row block: each step's sums start from zero and
// are folded with their own group's scales (after step 0 and at the block's end); HF: those
// scales in f32 (else bf16).
template <int BK, bool GRP, bool FB = false, bool H = false, bool HF = false>
__global__ __launch_bounds__(kThreads) void qdense_gemm_kernel(GemmArgs a) {
  static_assert(!H || (GRP && FB), "32-row groups: the fold-every-step form");
  static_assert(!HF || H, "f32 scales for 32-row groups only");
  constexpr int PF = kPf;
  // With scale groups the tile is 256 x 64: each wave keeps two of the four interleaved MFMA
  // column sets (columns 4*cg + 2*wc + c, c = 0, 1), which halves both accumulator sets so that
  // the second one fits beside the operands without spilling.
  constexpr int BN = kBN;
  constexpr int NC = 4;  // MFMA column sets per wave
  static_assert(kUnroll % PF == 0, "register slots cycle within the unroll");
  // Tile order: consecutive work items go to one XCD (workgroups are dispatched round-robin over
  // the 8); with whole 2 x 16 tile groups, 32 consecutive items form one group.  DotGeneral
  // batches are consecutive runs of items.
  const int bid = blockIdx.x;
  const int whole = a.split_from;  // whole-tile work items (dispatched first)
  int item, half = -1;
  if (bid < whole) {
    item = (whole & 7) == 0 ? (bid & 7) * (whole >> 3) + (bid >> 3) : bid;
  } else {
    item = whole + ((bid - whole) >> 1);
    half = (bid - whole) & 1;
  }
  const int batch = item / a.tiles;
  item -= batch * a.tiles;
  if constexpr (kDotB<BK>) {
    a.x += (size_t)batch * a.M * a.K;
    a.w += (size_t)batch * a.K * a.N * 2;
    a.out = (char*)a.out + (size_t)batch * a.M * a.N * (a.out_dt == MX_DTYPE_FLOAT32 ? 4 : 2);
  }
  int tm, tn;
  if (a.grouped) {
    const int g = item >> 5, q = item & 31, gpr = a.tiles_n >> 4;
    tm = 2 * (g / gpr) + (q >> 4);
    tn = 16 * (g % gpr) + (q & 15);
  } else {
    tm = item / a.tiles_n;
    tn = item % a.tiles_n;
  }
  const int m0 = tm * kBM, n0 = tn * BN;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wr = wave & 3, wc = wave >> 2;
  const int cg = lane & 15, kq = lane >> 4;
  const size_t N = (size_t)a.N;
  const int lda = a.K;  // x row stride
  if constexpr (!kDotB<BK>) {
    if (half >= 0) {
      // This workgroup's half of K: the operands start at its first 64-row block (a whole
      // number of scale groups, checked by the host) and K is the half's extent.
      const int kbeg = half * (a.K / kBK / 2);
      a.x += (size_t)kbeg * kBK;
      a.w += k4B<BK> ? (size_t)kbeg * kBK * N / 2 : (size_t)kbeg * kBK * N;
      if (a.gpb > 0)
        a.scale = (const char*)a.scale + (size_t)(kbeg / a.gpb) * (H ? 2 : 1) * N * (a.s_dt == MX_DTYPE_FLOAT32 ? 4 : 2);
      a.K /= 2;
    }
  }
  const int KB = a.K / kBK;

  constexpr int XB = kXBufs<BK, GRP, FB>;
  __shared__ __attribute__((aligned(16))) uint8_t xs[XB][kABytes];
  __shared__ __attribute__((aligned(16))) uint8_t bt[2][kBtBytes];

  // x: each wave moves kXDma 1 KB pieces of a block straight into LDS: piece q = kXDma*wave + i
  // holds rows 8q .. 8q + 7 (128 bytes each); lane l lands at row 8q + l / 8, 16-byte slot
  // l % 8, which holds the row's k-chunk (l % 8) ^ ((row >> 1) & 7).  Rows past M read row M-1.
  const int t = threadIdx.x;
  // Byte offsets from the block's start in x (M * K < 2^31 elements, checked by the host).
  uint32_t xoff[kXDma];
#pragma unroll
  for (int i = 0; i < kXDma; ++i) {
    const int r = 8 * (kXDma * wave + i) + (lane >> 3);
    xoff[i] = 2u * ((uint32_t)min(m0 + r, a.M - 1) * (uint32_t)lda + 8u * ((lane & 7) ^ ((r >> 1) & 7)));
  }
  const uint32_t xs_lds = lds_addr(&xs[0][0]) + (uint32_t)(kXDma * wave) * 1024u;
  auto dma_x = [&](int kb) {
    const uint32_t dst = xs_lds + (uint32_t)(kb % XB) * kABytes;
    kb = min(kb, KB - 1);
#pragma unroll
    for (int i = 0; i < kXDma; ++i) lds_dma_b128(a.x + (size_t)kb * kBK, xoff[i], dst + 1024u * i);
  };
  // B, [K, N] kinds: thread t (cq = t % 32, j = t / 32) converts columns 4*cq .. 4*cq + 3 and
  // rows 4*j .. 4*j + 3 of each block; the 32 threads of a j read one contiguous row segment
  // (128 bytes of int8, 64 of 4-bit, 256 of a half type).  Columns past N read column 0 (their
  // outputs are not stored).
  // [N, K] kinds: B rows are k-contiguous like x: thread t copies 16-byte chunks q = t + kThreads*i,
  // column q / 8 (rows past N read row N-1), k-chunk q % 8.
  constexpr int kCQ = 32, kJ = kThreads / kCQ;  // threads per row group, row groups of one block
  static_assert(4 * kJ == kBK && 4 * kCQ == kBN, "B conversion split");
  const int cq = t % kCQ, j = t / kCQ;
  const int wcol = n0 + 4 * cq + 4 <= a.N ? n0 + 4 * cq : 0;
  const uint8_t* wsrc = k4B<BK> ? a.w + ((size_t)(4 * j) * N + wcol) / 2
                                : a.w + ((size_t)(4 * j) * N + wcol) * (kDotB<BK> ? 2 : 1);
  // Column 4*cq + c lives in Bt row (4*cq + c) ^ (cq & 1), k-chunk j / 2 swizzled by (cq / 2) & 7,
  // 8-byte half j % 2 of the chunk.
  const uint32_t cv_off = (uint32_t)((((j >> 1) ^ ((cq >> 1) & 7)) << 4) + ((j & 1) << 3));
  constexpr int kNKLoads = kBtBytes / (kThreads * 16);
  const uint8_t* nksrc[kNKLoads];
  uint32_t nkdst[kNKLoads];
  if constexpr (kNKB<BK>) {
#pragma unroll
    for (int i = 0; i < kNKLoads; ++i) {
      const int q = t + kThreads * i;
      const int r = q >> 3, c = q & 7, p = r ^ ((r >> 2) & 1);
      nksrc[i] = a.w + ((size_t)min(n0 + r, a.N - 1) * a.K + 8 * c) * 2;
      nkdst[i] = (uint32_t)(p * (kBK * 2) + ((c ^ ((p >> 3) & 7)) << 4));
    }
  }
  // Register words of one block of B per thread.
  constexpr int kWWords = kNKB<BK> ? 4 * kNKLoads : (kDotB<BK> ? 2 * kWLoads : kWLoads);
  constexpr int kWWrites = kNKB<BK> ? kNKLoads : 4;  // Bt writes per thread per block
  auto load_w = [&](int kb, uint32_t (&dst)[kWWords]) {
    kb = min(kb, KB - 1);
    if constexpr (kNKB<BK>) {
#pragma unroll
      for (int i = 0; i < kNKLoads; ++i) {
        const u32x4_v v = __builtin_nontemporal_load((const u32x4_v*)(nksrc[i] + (size_t)kb * kBK * 2));
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[4 * i + e] = v[e];
      }
    } else if constexpr (kDotB<BK>) {
#pragma unroll
      for (int e = 0; e < kWLoads; ++e) {
        const u32x2_v v = __builtin_nontemporal_load((const u32x2_v*)(wsrc + (size_t)(kb * kBK + e) * N * 2));
        dst[2 * e] = v[0];
        dst[2 * e + 1] = v[1];
      }
    } else if constexpr (k4B<BK>) {
#pragma unroll
      for (int e = 0; e < kWLoads; ++e)
        dst[e] = __builtin_nontemporal_load((const uint16_t*)(wsrc + (size_t)(kb * kBK + e) * (N / 2)));
    } else {
#pragma unroll
      for (int e = 0; e < kWLoads; ++e)
        dst[e] = __builtin_nontemporal_load((const uint32_t*)(wsrc + (size_t)(kb * kBK + e) * N));
    }
  };
  // Four k-values of each of four consecutive columns (Bt rows 128 bytes apart): int8 and 4-bit
  // converted exactly to bf16, half values regrouped by column.  [N, K]: the chunks as loaded.
  auto store_w = [&](const uint32_t (&w4)[kWWords], int buf) {
    if constexpr (kNKB<BK>) {
#pragma unroll
      for (int i = 0; i < kNKLoads; ++i)
        *(u32x4_v*)(&bt[buf][nkdst[i]]) = u32x4_v{w4[4 * i], w4[4 * i + 1], w4[4 * i + 2], w4[4 * i + 3]};
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        u32x2_v v;
        if constexpr (kDotB<BK>) {
          // Row e holds columns 0..3 as dwords [c0 c1][c2 c3]; column c's k-pairs (e, e+1).
          const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
          v = u32x2_v{__builtin_amdgcn_perm(w4[2 * 1 + (c >> 1)], w4[2 * 0 + (c >> 1)], sel),
                      __builtin_amdgcn_perm(w4[2 * 3 + (c >> 1)], w4[2 * 2 + (c >> 1)], sel)};
        } else {
          float f[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (BK == kBI8)
              f[e] = (float)(int8_t)(w4[e] >> (8 * c));
            else if constexpr (BK == kBU8)
              f[e] = (float)(uint8_t)(w4[e] >> (8 * c));
            else if constexpr (BK == kBI4)  // nibble c, low nibble first (reference packing)
              f[e] = (float)((int32_t)(w4[e] << (28 - 4 * c)) >> 28);
            else
              f[e] = (float)((w4[e] >> (4 * c)) & 15u);
          }
          v = u32x2_v{__builtin_amdgcn_perm(__float_as_uint(f[1]), __float_as_uint(f[0]), 0x07060302u),
                      __builtin_amdgcn_perm(__float_as_uint(f[3]), __float_as_uint(f[2]), 0x07060302u)};
        }
        *(u32x2_v*)(&bt[buf][cv_off + (uint32_t)((4 * cq + (c ^ (cq & 1))) * (kBK * 2))]) = v;
      }
    }
  };

  // acc: the total; accg: the current scale group's sums (grouped scales only).
  f32x4_t acc[4][NC], accg[4][NC];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[rb][c] = accg[rb][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Grouped scales: this lane's 4 columns' scales of the group being summed, loaded a group ahead.
  // This lane's first column: 64*wc + 4*cg (four consecutive).
  const int lcol = n0 + 64 * wc + 4 * cg;
  const int scol = min(lcol, a.N - NC);
  float sg[NC];
  u32x2_v sgw = {0u, 0u}, sgw2 = {0u, 0u};
  f32x4_t sgf = {0.f, 0.f, 0.f, 0.f}, sgf2 = sgf;  // HF: the block's two rows of f32 scales
#pragma unroll
  for (int c = 0; c < NC; ++c) sg[c] = 0.f;
  auto load_sg = [&](int g) __attribute__((always_inline)) {
    g = min(g, a.K / (kBK * max(a.gpb, 1)) - 1);
    if constexpr (HF) {
      // The block's two scale rows (groups 2g and 2g + 1), one 16-byte load each.
      sgf = *(const f32x4_t*)((const float*)a.scale + (size_t)(2 * g) * N + scol);
      sgf2 = *(const f32x4_t*)((const float*)a.scale + (size_t)(2 * g + 1) * N + scol);
    } else if constexpr (H) {
      // The block's two scale rows (groups 2g and 2g + 1).
      sgw = *(const u32x2_v*)((const uint16_t*)a.scale + (size_t)(2 * g) * N + scol);
      sgw2 = *(const u32x2_v*)((const uint16_t*)a.scale + (size_t)(2 * g + 1) * N + scol);
    } else if constexpr (FB) {
      // bf16 scales (the host takes these kernels for bf16 scales only): one 8-byte load, kept
      // as loaded until the fold.
      sgw = *(const u32x2_v*)((const uint16_t*)a.scale + (size_t)g * N + scol);
    } else {
#pragma unroll
      for (int c = 0; c < NC; ++c) sg[c] = load_f(a.scale, (size_t)g * N + scol + c, a.s_dt);
    }
  };
  if constexpr (GRP) load_sg(0);

  // MFMA operands of one 32-row step: x row 64*wr + 16*rb + cg, Bt column 64*wc + 4*cg + c (Bt
  // row 64*wc + 4*cg + (c ^ (cg & 1))); with groups, Bt column 4*cg + 2*wc + c.
  const uint32_t a_row = (uint32_t)((64 * wr + cg) * (kBK * 2));
  const uint32_t b_col = (uint32_t)((64 * wc + 4 * cg) * (kBK * 2));
  const int b_par = cg & 1;
  // Operands of one 32-row step (sub = 0, 1 of a block) from LDS buffer buf, and its 16 MFMAs.
  auto read_step = [&](int xbuf, int buf, int sub, u32x4_v (&A)[4], u32x4_v (&B)[NC]) {
    const int kc = 4 * sub + kq;  // 16-byte k-chunk of this lane
    const uint8_t* ap = &xs[xbuf][a_row + ((kc ^ (cg >> 1)) << 4)];
    const uint8_t* bp = &bt[buf][b_col + ((kc ^ ((cg >> 1) & 7)) << 4)];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) A[rb] = *(const u32x4_v*)(ap + rb * 16 * (kBK * 2));
#pragma unroll
    for (int c = 0; c < NC; ++c) B[c] = *(const u32x4_v*)(bp + (c ^ b_par) * (kBK * 2));
  };
  auto mma_step = [&](const u32x4_v (&A)[4], const u32x4_v (&B)[NC], auto fresh) __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if constexpr (GRP && decltype(fresh)::value)
          accg[rb][c] = mfma<BK>(A[rb], B[c], f32x4_t{0.f, 0.f, 0.f, 0.f});
        else if constexpr (GRP)
          accg[rb][c] = mfma<BK>(A[rb], B[c], accg[rb][c]);
        else
          acc[rb][c] = mfma<BK>(A[rb], B[c], acc[rb][c]);
      }
  };
  // End of a scale group (every block with FB): acc += accg * s (this lane's columns; accg = 0
  // unless the next group's first MFMAs start from zero), then the scales of group g_next.
  // acc += accg * s with the bf16 scales of one loaded scale row (FB), or the f32 scales in sg.
  auto fold_sums = [&](const u32x2_v& w, const f32x4_t& wf) __attribute__((always_inline)) {
    if constexpr (HF) {
#pragma unroll
      for (int c = 0; c < NC; ++c) sg[c] = wf[c];
    } else if constexpr (FB) {
      sg[0] = __uint_as_float(w[0] << 16);
      sg[1] = __uint_as_float(w[0] & 0xFFFF0000u);
      sg[2] = __uint_as_float(w[1] << 16);
      sg[3] = __uint_as_float(w[1] & 0xFFFF0000u);
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[rb][c][r] = __builtin_fmaf(accg[rb][c][r], sg[c], acc[rb][c][r]);
        if constexpr (!FB) accg[rb][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
  };
  auto fold = [&](int g_next) __attribute__((always_inline)) {
    fold_sums(H ? sgw2 : sgw, sgf2);  // H: the block's second group (its first was folded after step 0)
    load_sg(g_next);
  };

  // x moves by direct-to-LDS loads XB - 1 blocks ahead of its use (XB buffers: block kb's
  // buffer takes block kb + XB once its last operands are read, i.e. after block kb's barrier).
  // w moves through register slots that hold the next PF blocks (slot b % PF holds block b from
  // its load during block b - PF to its conversion during block b - 2) and is converted into the
  // Bt buffer that block kb leaves after its barrier (Bt buffers alternate, block b in buffer
  // b % 2).  Step 0 of block kb reads step 1's operands under its MFMAs; then each wave waits for
  // its own x loads of block kb + 1 and the barrier publishes that block (x and Bt) and retires
  // the reads of block kb.  Step 1 reads block kb + 1's step-0 operands, converts and writes block
  // kb + 2's weights, and issues the loads of blocks kb + PF (w) and kb + XB (x), all under its
  // MFMAs.  Every step issues its loads in one order (w, then x), so the number of loads issued
  // after a block's x loads is fixed: (XB - 2) * (kWGl + kXDma) when that block is published.  The weights'
  // conversion waits for loads two blocks old, and the compiler's count of them (it does not see
  // the x loads) only adds x loads at least as old as the ones the barrier needs.
  // (sched_barrier keeps the compiler from regrouping the phases.)
  constexpr int kWGl = kNKB<BK> ? kNKLoads : kWLoads;
  static_assert(PF >= 3 && kUnroll % PF == 0, "a block's weights are converted two blocks after their load");
  uint32_t wr4[PF][kWWords];
  u32x4_v A0[4], B0[NC], A1[4], B1[NC];
  int g_left = a.gpb, g_idx = 0;  // scale groups: blocks left in the current group, its index
  auto block = [&](int kb, auto step) __attribute__((always_inline)) {
    constexpr int U = decltype(step)::value;  // kb % kUnroll
    constexpr int S = U % PF, S2 = (U + 2) % PF, B = U % 2;
    const int xb = (int)((unsigned)kb % XB), xb1 = xb == XB - 1 ? 0 : xb + 1;
    // FB: the block's first step starts its sums from zero (the C operand 0).
    using Fresh = std::integral_constant<bool, FB>;
    using Acc = std::integral_constant<bool, false>;
    read_step(xb, B, 1, A1, B1);
    mma_step(A0, B0, Fresh{});
#pragma unroll
    for (int i = 0; i < 4 + NC; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (H) {
      fold_sums(sgw, sgf);  // the block's first 32-row group
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vm<(XB - 2) * (kWGl + kXDma)>();  // this wave's x loads of block kb + 1 are in LDS
    lds_barrier();
    read_step(xb1, B ^ 1, 0, A0, B0);
    store_w(wr4[S2], B);
    load_w(kb + PF, wr4[S]);
    dma_x(kb + XB);
    mma_step(A1, B1, std::integral_constant<bool, H>{});  // H: the second group starts from zero
#pragma unroll
    for (int i = 0; i < 4 + NC; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    }
#pragma unroll
    for (int i = 0; i < kWWrites; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    }
#pragma unroll
    for (int i = 0; i < kWGl; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (GRP && FB) {
      // Every block's sums are folded with its group's scales; the scale row of the next block
      // advances every a.gpb blocks (scalar countdown, no branch).
      const int last = --g_left == 0;
      g_left = last ? a.gpb : g_left;
      g_idx += last;
      fold(g_idx);
      __builtin_amdgcn_sched_barrier(0);
    } else if constexpr (GRP) {
      if (--g_left == 0) {
        g_left = a.gpb;
        fold(++g_idx);
      }
    }
  };
  auto blocks = [&](int kb, int n, auto... steps) { ((steps.value < n ? block(kb + steps.value, steps) : void()), ...); };

  // Prologue: the loads of blocks 0..PF-1 (w) and 0..XB-1 (x), all waited for; blocks 0 and 1's
  // weights into their Bt buffers.
#pragma unroll
  for (int p = 0; p < PF; ++p) load_w(p, wr4[p]);
#pragma unroll
  for (int p = 0; p < XB; ++p) dma_x(p);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  store_w(wr4[0], 0);
  store_w(wr4[1], 1);
  lds_barrier();
  read_step(0, 0, 0, A0, B0);
  int kb = 0;
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  static_assert(kUnroll == 4, "unrolled steps");
  for (; kb + kUnroll <= KB; kb += kUnroll) blocks(kb, kUnroll, I0{}, I1{}, I2{}, I3{});
  blocks(kb, KB - kb, I0{}, I1{}, I2{});

  if constexpr (!kDotB<BK>) {
    if (half >= 0) {
      // Split tail: store this half's sums, count the arrival; the second to arrive adds the
      // other half's sums in the order half 0 + half 1 and goes on to the epilogue.  The partial
      // tiles are stored and loaded with the agent-scope coherence bit (sc1); the two halves run
      // on different XCDs.
      // The arrival flag takes the first word of a Bt buffer: every wave has left the main loop
      // (the barrier below comes first), and four x buffers leave no LDS beyond the two.
      int& s_last = *(int*)&bt[0][0];
      const int tt = item - whole;  // tail tile
      const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
          a.part + (size_t)tt * 2 * 16 * kThreads * 4, (short)0, 2 * 16 * kThreads * 16, 0x00020000);
      constexpr int kSc1 = 16;
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int c = 0; c < NC; ++c)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_v, acc[rb][c]), prs,
                                                (unsigned)(((half * 16 + 4 * rb + c) * kThreads + t) * 16), 0, kSc1);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (t == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&a.ctr[tt], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == 1u) __hip_atomic_store(&a.ctr[tt], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == 1u;
      }
      __syncthreads();
      if (!s_last) return;
      const int other = half ^ 1;
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const f32x4_t o = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                            prs, (unsigned)(((other * 16 + 4 * rb + c) * kThreads + t) * 16), 0, kSc1));
          acc[rb][c] = half == 0 ? acc[rb][c] + o : o + acc[rb][c];
        }
    }
  }

  // Epilogue: y = act(acc * s[n] + bias[n]) for this lane's 4 columns (DotGeneral: the f32 sums,
  // or the sums rounded to the half output dtype as ConvertDType rounds them, 4 columns per store).
  const int ncol = lcol;
  if (ncol >= a.N) return;
  if constexpr (kDotB<BK>) {
    const int r0 = m0 + 64 * wr + 4 * kq;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = r0 + 16 * rb + r;
        if (row >= a.M) continue;
        const size_t o = (size_t)row * N + ncol;
        if (a.out_dt == MX_DTYPE_FLOAT32) {
          *(f32x4_t*)((float*)a.out + o) = f32x4_t{acc[rb][0][r], acc[rb][1][r], acc[rb][2][r], acc[rb][3][r]};
        } else {
          uint32_t h[4];
#pragma unroll
          for (int c = 0; c < 4; ++c)
            h[c] = a.out_dt == MX_DTYPE_BFLOAT16 ? f32_to_bf16(acc[rb][c][r]) : f32_to_f16(acc[rb][c][r]);
          *(u32x2_v*)((uint16_t*)a.out + o) = u32x2_v{h[0] | h[1] << 16, h[2] | h[3] << 16};
        }
      }
    return;
  } else {
    float sc[4], bi[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      sc[c] = GRP ? 1.0f : load_f(a.scale, ncol + c, a.s_dt);  // grouped: applied by fold()
      bi[c] = a.bias ? load_f(a.bias, ncol + c, a.b_dt) : 0.0f;
    }
    const int row0 = m0 + 64 * wr + 4 * kq;
    uint16_t* out = (uint16_t*)a.out;
    switch (a.act) {
      case MX_ACT_GELU: store_tile<MX_ACT_GELU>(acc, sc, bi, out, row0, a.M, N, ncol); break;
      case MX_ACT_RELU: store_tile<MX_ACT_RELU>(acc, sc, bi, out, row0, a.M, N, ncol); break;
      case MX_ACT_SILU: store_tile<MX_ACT_SILU>(acc, sc, bi, out, row0, a.M, N, ncol); break;
      case MX_ACT_HARDSWISH: store_tile<MX_ACT_HARDSWISH>(acc, sc, bi, out, row0, a.M, N, ncol); break;
      case MX_ACT_TANH: store_tile<MX_ACT_TANH>(acc, sc, bi, out, row0, a.M, N, ncol); break;
      default: store_tile<MX_ACT_NONE>(acc, sc, bi, out, row0, a.M, N, ncol); break;
    }
  }
}

}  // namespace

bool qdense_gemm_fits(const QDenseDesc& d) {
  auto aligned = [](const void* p, size_t al) { return ((uintptr_t)p % al) == 0; };
  const bool per_channel = d.block_axis == 0 && d.block_size >= d.K;
  // Scale groups of whole 64-row blocks that tile K exactly, or groups of 32 rows (two per
  // block).  The group kernels load a lane's four scales as one vector (bf16: 8 bytes, f32 groups
  // of 32: 16 bytes), from a 16-byte-aligned scale array.
  const bool grouped = d.block_axis == 0 && d.block_size < d.K && d.K % d.block_size == 0 &&
                       (d.block_size % kBK == 0 || d.block_size == 32) &&
                       (aligned(d.scale, 16) || (d.s_dt == MX_DTYPE_FLOAT32 && d.block_size != 32));
  const bool wt = d.w_dt == MX_DTYPE_INT8 || d.w_dt == MX_DTYPE_UINT8 || d.w_dt == MX_DTYPE_INT4 ||
                  d.w_dt == MX_DTYPE_UINT4;
  return d.M > 16 && d.x_dt == MX_DTYPE_BFLOAT16 && d.scheme == MX_QUANT_LINEAR && !d.zp && (per_channel || grouped) &&
         wt && d.K >= kBK && d.K % kBK == 0 && d.N >= 16 && d.N % 16 == 0 && d.M < (1 << 30) && d.K < (1 << 30) &&
         d.N < (1 << 30) && d.M * d.K < ((int64_t)1 << 31) && aligned(d.w, 16) && aligned(d.x, 16) &&
         aligned(d.out, 16);
}

int qdense_gemm_run(mx_backend* b, const QDenseDesc& d, const char* name) {
  GemmArgs ga;
  ga.x = (const uint16_t*)d.x;
  ga.w = (const uint8_t*)d.w;
  ga.scale = d.scale;
  ga.bias = d.bias;
  ga.out = d.out;
  ga.M = (int)d.M;
  ga.K = (int)d.K;
  ga.N = (int)d.N;
  ga.s_dt = d.s_dt;
  ga.b_dt = d.b_dt;
  ga.act = d.act;
  const bool grouped = d.block_size < d.K;
  // The kernel's tile width: 64 for 4-bit weights with scale groups.
  const int64_t bn = kBN;
  const int64_t tiles_m = (d.M + kBM - 1) / kBM, tiles_n = (d.N + bn - 1) / bn;
  if (tiles_m * tiles_n > (int64_t)1 << 30)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: output too large for the GEMM path");
  ga.tiles_n = (int)tiles_n;
  ga.grouped = (tiles_m % 2 == 0 && tiles_n % 16 == 0) ? 1 : 0;
  ga.tiles = (int)(tiles_m * tiles_n);
  // Groups of 32 rows (bf16 scales): one block per pair of groups, each step folded on its own.
  const bool half = grouped && d.block_size == 32;
  ga.gpb = half ? 1 : grouped ? (int)(d.block_size / kBK) : 0;
  // Split tail: when the tiles leave a last partial round of at most half the CUs (planned for
  // MI355X's 256 CUs whatever the device reports, so the summation order depends on the shape
  // only), those tiles are computed as two halves of K by twice as many workgroups.  Not under
  // mx_qdense_noalloc (its static scratch is smaller than the partial tiles).
  const int64_t tiles = tiles_m * tiles_n, tail = tiles % kSplitPlanCUs;
  const int64_t KB = d.K / kBK;
  const bool split = tiles > kSplitPlanCUs && tail > 0 && 2 * tail <= kSplitPlanCUs && KB % 2 == 0 && KB >= 8 &&
                     (!grouped || (KB / 2) % ga.gpb == 0) && !b->noalloc_active;
  ga.split_from = (int)(split ? tiles - tail : tiles);
  ga.part = nullptr;
  ga.ctr = nullptr;
  if (split) {
    const size_t counter_bytes = 64 * 1024;  // shared with the decode kernels' counters (zero between launches)
    void* scratch = nullptr;
    MX_TRY(ensure_scratch(b, counter_bytes + (size_t)tail * 2 * 16 * kThreads * 16, &scratch));
    ga.ctr = (uint32_t*)scratch;
    ga.part = (float*)((char*)scratch + counter_bytes);
  }
  const int grid = (int)(split ? tiles + tail : tiles);
  hipStream_t st = b->stream;
  // bf16 group scales: the fold-every-block kernel; f32 group scales count blocks at run time.
  auto grouped_kernel = [&](auto kind) {
    constexpr int BK = decltype(kind)::value;
    if (half && d.s_dt == MX_DTYPE_FLOAT32)
      dispatch(qdense_gemm_kernel<BK, true, true, true, true>, grid, kThreads, 0, st, ga);
    else if (half)
      dispatch(qdense_gemm_kernel<BK, true, true, true>, grid, kThreads, 0, st, ga);
    else if (d.s_dt == MX_DTYPE_BFLOAT16)
      dispatch(qdense_gemm_kernel<BK, true, true>, grid, kThreads, 0, st, ga);
    else
      dispatch(qdense_gemm_kernel<BK, true>, grid, kThreads, 0, st, ga);
  };
  return launch(b, name, [&] {
    switch (d.w_dt) {
      case MX_DTYPE_INT8:
        grouped ? grouped_kernel(std::integral_constant<int, kBI8>{})
                : dispatch(qdense_gemm_kernel<kBI8, false>, grid, kThreads, 0, st, ga);
        break;
      case MX_DTYPE_UINT8:
        grouped ? grouped_kernel(std::integral_constant<int, kBU8>{})
                : dispatch(qdense_gemm_kernel<kBU8, false>, grid, kThreads, 0, st, ga);
        break;
      case MX_DTYPE_INT4:
        grouped ? grouped_kernel(std::integral_constant<int, kBI4>{})
                : dispatch(qdense_gemm_kernel<kBI4, false>, grid, kThreads, 0, st, ga);
        break;
      default:
        grouped ? grouped_kernel(std::integral_constant<int, kBU4>{})
                : dispatch(qdense_gemm_kernel<kBU4, false>, grid, kThreads, 0, st, ga);
        break;
    }
  });
}

// DotGeneral on the matrix cores: half-precision inputs, f32 sums (the lowering's accumulator,
// dot/dot.go:340-372), normalized [batch][M, K] x [batch][K, N] or [batch][N, K], stored as f32
// or rounded to the input's half dtype (the lowering's ConvertDType back, folded in).  Only the
// summation order differs from a sequential f32 sum (every half product is exact in f32).
bool dot_mfma_fits(const DotDesc& d) {
  auto aligned = [](const void* p, size_t al) { return ((uintptr_t)p % al) == 0; };
  const bool half = d.in_dt == MX_DTYPE_BFLOAT16 || d.in_dt == MX_DTYPE_FLOAT16;
  return half && (d.out_dt == MX_DTYPE_FLOAT32 || d.out_dt == d.in_dt) && d.M >= 1 && d.K >= kBK && d.K % kBK == 0 && d.N >= 16 &&
         d.N % 16 == 0 && d.B * d.M * d.N * d.K >= ((int64_t)1 << 24) && d.M < (1 << 30) && d.K < (1 << 30) &&
         d.N < (1 << 30) && d.M * d.K < ((int64_t)1 << 31) && aligned(d.lhs, 16) && aligned(d.rhs, 16) &&
         aligned(d.out, 16);
}

int dot_mfma_run(mx_backend* b, const DotDesc& d, const char* name) {
  GemmArgs ga{};
  ga.x = (const uint16_t*)d.lhs;
  ga.w = (const uint8_t*)d.rhs;
  ga.out = d.out;
  ga.out_dt = d.out_dt;
  ga.M = (int)d.M;
  ga.K = (int)d.K;
  ga.N = (int)d.N;
  const int64_t tiles_m = (d.M + kBM - 1) / kBM, tiles_n = (d.N + kBN - 1) / kBN;
  if (d.B * tiles_m * tiles_n > (int64_t)1 << 30)
    return set_error(MX_ERR_INVALID, "DotGeneral: output too large for the matrix-core path");
  ga.tiles_n = (int)tiles_n;
  ga.grouped = (tiles_m % 2 == 0 && tiles_n % 16 == 0) ? 1 : 0;
  ga.tiles = (int)(tiles_m * tiles_n);
  const int grid = (int)(d.B * tiles_m * tiles_n);
  ga.split_from = grid;  // DotGeneral: whole tiles only
  hipStream_t st = b->stream;
  const bool f16 = d.in_dt == MX_DTYPE_FLOAT16;
  return launch(b, name, [&] {
    if (d.rhs_transposed) {
      if (f16)
        dispatch(qdense_gemm_kernel<kBF16NK, false>, grid, kThreads, 0, st, ga);
      else
        dispatch(qdense_gemm_kernel<kBBf16NK, false>, grid, kThreads, 0, st, ga);
    } else {
      if (f16)
        dispatch(qdense_gemm_kernel<kBF16KN, false>, grid, kThreads, 0, st, ga);
      else
        dispatch(qdense_gemm_kernel<kBBf16KN, false>, grid, kThreads, 0, st, ga);
    }
  });
}

}  // namespace mx
