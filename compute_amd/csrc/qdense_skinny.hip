// Skinny FusedQuantizedDense on gfx950: decode and small-batch shapes (M <= 16 rows of bf16
// activations), weights [K, N] in Int8 / Uint8 / Int4 / Uint4 (reference packing), scales
// blocked along K (one scale per group of G rows and output column, or per output column).
//
// Reference semantics: quantizedDenseLinearInt (internal/gobackend/fusedops/quantizeddense.go:
// 616-650) then the activation epilogue (fusedops/dense.go:176-205), with the weight-group
// scale factored out of each group's partial sum:  y[m,n] = act(bias[n] +
//   sum_g s[g,n] * sum_{k in g} x[m,k] * w[k,n]).
// The products x*w are exact in f32 (bf16 x, |w| <= 255), so only the summation order differs
// from the reference loop.
//
// The kernel is HBM-bound: every weight byte is read once.  Each wave walks its T steps of 32 K
// rows in a software pipeline with two steps in flight: as soon as a step has been computed, the
// step two ahead is requested into the registers it used.  A step is dequantised in registers
// into the B operand of v_mfma_f32_16x16x32_bf16 (the matrix cores do the multiply-adds, the VALU
// only converts); the 16 rows of the A operand are the rows of x (rows >= M repeat row M-1 and
// are never stored).  The code is kept short on purpose: a launch this brief runs its
// instructions cold, so the main loop is a rolled loop (its body two steps, the last two steps
// peeled so that every iteration issues the same loads and each wait is exact) and the output
// code is one rolled loop with a short path for outputs without activation, pair or elementwise
// operand.
//
// Lane layout (wave of 64 lanes, cg = lane % 16, kq = lane / 16).  A lane reads 8 bytes of each
// of the rows k0 + 8*kq + e (e = 0..7) of a 32-row step: 16 int4 or 8 int8 columns (CPL), so a
// wave covers 16*CPL columns (256 or 128) and each row segment a wave reads is 128 contiguous
// bytes.  MFMA number c takes column col0 + c from every lane, so its result column j = cg is
// column CPL*j + c of the block, and the lane ends up holding rows 4*kq + r (r = 0..3) of its
// own CPL columns.
//
// Dequantisation into bf16 pairs (two K rows of one column per dword):
//   int8/uint8: exact conversion through f32 (a byte has at most 8 significant bits; the signed
//               byte is selected and sign-extended by the conversion itself), the two high
//               halves packed with one v_perm;
//   int4/uint4: v_perm gathers the bytes of two rows, then one and-xor (v_bitop3) turns a
//               nibble u into the bf16 bit pattern 0x4300|u = 128 + u (exact); for Int4 the same
//               xor flips bit 3 of the nibble, giving 136 + w.  The offset is removed once per
//               group with the group's row sums of x, which one extra MFMA against an all-ones B
//               operand produces.
//
// Work decomposition.  The K steps of a column block are dealt out T at a time to waves, in
// order; a workgroup of NW = 8 waves (7 or 4 for one row when 8-wave workgroups would leave a
// quarter of the CUs idle) takes NW consecutive wave-chunks (one K slice), so a column block has
// S = ceil(K/32 / (T*NW)) slices.  T is chosen per shape (the smallest even
// divisor of K/32 that keeps the grid within one workgroup per CU).  A wave folds a group's
// partial sums into its total with the group's scale when the group ends, or at its last step.
// The waves' partial tiles are summed through LDS in wave order; with S > 1 every workgroup
// stores its tile to scratch and the last one to arrive for the column block adds the S tiles in
// slice order (deterministic), adds the bias, applies the activation and rounds to bf16.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "device_common.h"
#include "mxrt_internal.h"

namespace mx {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_v __attribute__((ext_vector_type(2)));

constexpr int kSkMaxRows = 16;
constexpr int kSkWaves = 8;
constexpr int kSkLaneBytes = 8;  // bytes of one weight row per lane
constexpr int kSkPlanCUs = 256;  // CUs the work split is planned for (MI355X)

struct SkinnyArgs {
  const uint16_t* x;    // [M, K] bf16
  const uint8_t* w;     // [K, N] storage bytes
  const void* scale;    // [ceil(K/G), N]
  const void* bias;     // [N] or null
  uint16_t* out;        // [M, N] bf16
  float* partial;       // [S, M, N] (S > 1)
  uint32_t* counters;   // [column blocks], zero between launches
  const void* res;      // [M, N] epilogue operand (res_op != 0)
  // Pair mode: a second product over the same x (w2, scale2, bias2, act2: same shapes and
  // dtypes), out = round(round(act(y + bias)) * round(act2(y2 + bias2))).
  const uint8_t* w2;
  const void* scale2;
  const void* bias2;
  int M, K, N;
  int FS;  // K steps (32 rows) per scale group; K/32 for one scale per output column
  int T;   // K steps per wave (the host makes K/32 a multiple of T)
  int S, act, b_dt, res_dt, res_op;
  int pair, act2, b2_dt;
};

__device__ __forceinline__ f32x4_t sk_mfma(const u32x4_v& a, const u32x4_v& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}

// A uniform constant held in a VGPR: (t & mask) | c then selects one v_and_or_b32 (a VOP3
// instruction takes no literal and at most one scalar operand here).
__device__ __forceinline__ uint32_t vgpr_const(uint32_t x) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "s"(x));
  return r;
}

// Workgroup index -> work item, so that the S slices of one column block (consecutive items)
// run on one XCD and share its L2: workgroups are dispatched round-robin over the 8 XCDs, and
// each XCD takes a contiguous run of items (any grid size).
__device__ __forceinline__ int sk_xcd_swizzle(int bid, int total) {
  // XCD x receives workgroups x, x + 8, ...: total / 8 of them, one more when x < total % 8.
  const int x = bid & 7, base = total >> 3, rem = total & 7;
  return x * base + min(x, rem) + (bid >> 3);
}

// Elements idx .. idx + 3 of a bf16 or f32 array (idx % 4 == 0, the array 16-byte aligned: one
// 8- or 16-byte load), issued by sk_quad_load and converted once arrived by sk_quad_value.
__device__ __forceinline__ u32x4_v sk_quad_load(const void* p, size_t idx, int dt) {
  if (dt == MX_DTYPE_BFLOAT16) {
    const u32x2_v v = *(const u32x2_v*)((const uint16_t*)p + idx);
    return u32x4_v{v[0], v[1], 0u, 0u};
  }
  return *(const u32x4_v*)((const float*)p + idx);
}

__device__ __forceinline__ f32x4_t sk_quad_value(const u32x4_v& w, int dt) {
  if (dt == MX_DTYPE_BFLOAT16)
    return f32x4_t{__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xFFFF0000u), __uint_as_float(w[1] << 16),
                   __uint_as_float(w[1] & 0xFFFF0000u)};
  return __builtin_bit_cast(f32x4_t, w);
}

// WDT: weight dtype.  MR: rows of the MFMA result kept per lane (1 when M == 1, else 4).
// SF32: f32 scales (else bf16).  PIPE: T is even and two steps are in flight per wave (else
// T == 1).  The main loop is a rolled loop whose body is two steps, so the code a CU fetches
// stays small: a kernel this short-lived runs its instructions cold, and every instruction-cache
// line it misses costs a trip to L2 or beyond.
// G2: the scale groups are two steps (G = 64), so a group is exactly one loop iteration's pair:
// its first step's MFMAs start from zero and its second folds, with no clearing of the sums.
// WV: waves per workgroup, 8, or 7 or 4 for single-row launches whose 8-wave grid would leave a
// quarter of the CUs idle (7: one workgroup per CU; 4: twice the workgroups, up to two per CU).
// XT (T = XT = 4 steps per wave, all of them in one scale group): the wave's scale row is loaded
// once, ahead of its first weights, and with one row of x (MR == 1) the wave's 128 values of x
// as well, so that a step requests only its weights (and x for several rows).  C2: 9.71 ->
// 9.49 us per launch in an A/B on one box.
template <int WDT, int MR, bool SF32, bool PIPE, bool G2, int WV = kSkWaves, int XT = 0>
__global__ __launch_bounds__(64 * WV, 2) void qdense_skinny_kernel(const uint16_t* px, const uint8_t* pw,
                                                                   const void* pscale, int pK, int pN, int pT,
                                                                   int pFS, int pS, SkinnyArgs a) {
  a.x = px;
  a.w = pw;
  a.scale = pscale;
  a.K = pK;
  a.N = pN;
  a.T = pT;
  a.FS = pFS;
  a.S = pS;
  constexpr int kWv = WV, kThr = 64 * WV;
  constexpr bool kI4 = WDT == MX_DTYPE_INT4 || WDT == MX_DTYPE_UINT4;
  constexpr int CPL = kI4 ? 2 * kSkLaneBytes : kSkLaneBytes;  // columns per lane
  constexpr int kCols = 16 * CPL;                              // columns per workgroup
  constexpr int kSLoads = CPL * (SF32 ? 4 : 2) / 16;           // 16-byte scale loads per step
  constexpr float kOff = WDT == MX_DTYPE_INT4 ? 136.0f : (WDT == MX_DTYPE_UINT4 ? 128.0f : 0.0f);
  extern __shared__ __attribute__((aligned(16))) float red[];
  __shared__ int s_last;

  const int item = sk_xcd_swizzle(blockIdx.x, gridDim.x);
  // Work items of a column block are consecutive slices.  In pair mode a workgroup computes its
  // slice of both products, one after the other, each summed exactly as its own launch sums it.
  const int NM = a.pair ? 2 : 1;
  const int SP = NM * a.S;  // partial tiles per column block, [matrix][slice]
  const int cb = item / a.S, slice = item % a.S;
  // The wave index is wave-uniform; saying so keeps the control flow scalar.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int cg = lane & 15, kq = lane >> 4;
  const int KS = a.K >> 5;
  const int k0 = (slice * kWv + wave) * a.T;  // first K step of this wave
  const int cblk = cb * kCols;
  const int col0 = cblk + cg * CPL;

  const int M = a.M;
  constexpr int kQPR = kCols / 4;  // quads per tile row
  constexpr int kMaxQ = (kSkMaxRows * kQPR + kThr - 1) / kThr;  // quads per thread (M = 16)
  const int t = threadIdx.x;
  const int MC = M * kCols, NQ = M * kQPR;
  auto wave_sum = [&](int g) __attribute__((always_inline)) {
    f32x4_t y = *(const f32x4_t*)(red + 4 * g);
#pragma unroll
    for (int w = 1; w < kWv; ++w) y += *(const f32x4_t*)(red + w * MC + 4 * g);
    return y;
  };
  // The workgroup's tile of each product, summed over the waves (quad g = t + i * kThr):
  // the last product's stays as the waves' tiles in LDS, the first of a pair is summed into an
  // LDS tile of its own before the second is computed.
  float* held = red + (size_t)kWv * M * kCols;
  auto tile = [&](int mat, int i) __attribute__((always_inline)) {
    const int g = min(t + i * kThr, NQ - 1);
    return mat + 1 < NM ? *(const f32x4_t*)(held + 4 * g) : wave_sum(g);
  };
#pragma unroll 1
  for (int mat = 0; mat < NM; ++mat) {
  const uint8_t* wmat = mat ? a.w2 : a.w;
  const void* smat = mat ? a.scale2 : a.scale;
  float tot[CPL][MR];
  #pragma unroll
    for (int c = 0; c < CPL; ++c)
  #pragma unroll
      for (int r = 0; r < MR; ++r) tot[c][r] = 0.0f;
  
    if (k0 < KS) {
      // Lanes whose columns lie past N read column 0 instead (their results are never stored).
      const size_t row_bytes = kI4 ? (size_t)(a.N >> 1) : (size_t)a.N;
      const size_t lbyte = kI4 ? (size_t)(col0 >> 1) : (size_t)col0;
      const uint8_t* wp = wmat + (size_t)(8 * kq) * row_bytes + (lbyte + kSkLaneBytes <= row_bytes ? lbyte : 0);
      const uint16_t* xp = a.x + (size_t)min(cg, a.M - 1) * a.K + 8 * kq;
      const char* sp = (const char*)smat + (size_t)(col0 < a.N ? col0 : 0) * (SF32 ? 4 : 2);
      const size_t srow = (size_t)a.N * (SF32 ? 4 : 2);
      static_assert(XT == 0 || (XT == 4 && PIPE && !G2), "XT: four steps per wave");
      constexpr bool kXW = XT && MR == 1;  // x once per wave
      u32x4_v xw[kXW ? XT : 1], sw[XT ? kSLoads : 1];
      if constexpr (XT) {
        if constexpr (kXW) {
  #pragma unroll
          for (int q = 0; q < XT; ++q) xw[q] = *(const u32x4_v*)(xp + 32 * (k0 + q));
        }
        const char* sg0 = sp + (size_t)(k0 / a.FS) * srow;
  #pragma unroll
        for (int q = 0; q < kSLoads; ++q) sw[q] = *(const u32x4_v*)(sg0 + 16 * q);
      }
  
      // One step's operands: x (16 bytes), eight 8-byte weight row segments, and the scales of the
      // step's group (loaded with every step, so that every step issues the same loads and each
      // wait is exact; the repeats within a group hit the cache).
      struct Slot {
        u32x4_v x;
        u32x2_v w[8];
        u32x4_v s[kSLoads];
      };
      int ig = k0 / a.FS, irem = a.FS - k0 % a.FS;  // group and steps left in it, issue order
      // odd: the step's parity, known at each call site.  With two-step groups (G2) only the odd
      // step, which folds the group, needs the scales.
      auto issue = [&](Slot& sl, int k, auto odd) __attribute__((always_inline)) {
        if constexpr (!kXW) sl.x = *(const u32x4_v*)(xp + 32 * k);
        const uint8_t* wk = wp + (size_t)(32 * k) * row_bytes;
  #pragma unroll
        for (int e = 0; e < 8; ++e) sl.w[e] = __builtin_nontemporal_load((const u32x2_v*)(wk + (size_t)e * row_bytes));
        const char* sg = sp + (size_t)ig * srow;
  #pragma unroll
        for (int q = 0; q < kSLoads; ++q) {
          if constexpr (!XT && !(G2 && !decltype(odd)::value)) sl.s[q] = *(const u32x4_v*)(sg + 16 * q);
        }
        if (--irem == 0) {
          ++ig;
          irem = a.FS;
        }
      };
  
      // A nibble u (bits 0-3 and 16-19 after the mask) becomes the bf16 pattern 0x4300 | u =
      // 128 + u with one xor (the mask leaves no other bits); for Int4 the same xor also flips bit 3
      // of the nibble, giving 136 + w.  (x & m) ^ c is one v_bitop3_b32.
      const uint32_t kMask = 0x000F000Fu;
      const uint32_t kOr = vgpr_const(WDT == MX_DTYPE_INT4 ? 0x43084308u : 0x43004300u);
      const u32x4_v ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
      const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
      f32x4_t grp[CPL], sx = zero;
  #pragma unroll
      for (int c = 0; c < CPL; ++c) grp[c] = zero;
      // A step: dequantise into MFMA B operands and accumulate the group's partial sums.
      // xa: the step's x operand (the slot's, or with one row and XT the wave's x loaded at entry).
      auto compute = [&](const Slot& sl, const u32x4_v& xa, auto zc) __attribute__((always_inline)) {
        constexpr bool Z = decltype(zc)::value;  // the group's first step: sums start from zero
        if constexpr (kI4) {
  #pragma unroll
          for (int d = 0; d < CPL / 8; ++d) {
            uint32_t bq[8][4];  // columns 8d + 0..7, four pair-dwords each
  #pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
              const uint32_t A = sl.w[2 * pp][d], B = sl.w[2 * pp + 1][d];
              const uint32_t t0 = __builtin_amdgcn_perm(B, A, 0x06040200u);  // [A.b0, A.b2, B.b0, B.b2]
              const uint32_t t1 = __builtin_amdgcn_perm(B, A, 0x07050301u);  // [A.b1, A.b3, B.b1, B.b3]
              bq[0][pp] = (t0 & kMask) ^ kOr;
              bq[1][pp] = ((t0 >> 4) & kMask) ^ kOr;
              bq[4][pp] = ((t0 >> 8) & kMask) ^ kOr;
              bq[5][pp] = ((t0 >> 12) & kMask) ^ kOr;
              bq[2][pp] = (t1 & kMask) ^ kOr;
              bq[3][pp] = ((t1 >> 4) & kMask) ^ kOr;
              bq[6][pp] = ((t1 >> 8) & kMask) ^ kOr;
              bq[7][pp] = ((t1 >> 12) & kMask) ^ kOr;
            }
  #pragma unroll
            for (int c = 0; c < 8; ++c)
              grp[8 * d + c] = sk_mfma(xa, u32x4_v{bq[c][0], bq[c][1], bq[c][2], bq[c][3]}, Z ? zero : grp[8 * d + c]);
          }
          sx = sk_mfma(xa, ones, Z ? zero : sx);
        } else {
  #pragma unroll
          for (int d = 0; d < CPL / 4; ++d) {
  #pragma unroll
            for (int c = 0; c < 4; ++c) {
              uint32_t bq[4];
  #pragma unroll
              for (int pp = 0; pp < 4; ++pp) {
                const uint32_t r0 = sl.w[2 * pp][d], r1 = sl.w[2 * pp + 1][d];
                float f0, f1;
                if constexpr (WDT == MX_DTYPE_INT8) {
                  f0 = (float)(int8_t)(r0 >> (8 * c));
                  f1 = (float)(int8_t)(r1 >> (8 * c));
                } else {
                  f0 = (float)(uint8_t)(r0 >> (8 * c));
                  f1 = (float)(uint8_t)(r1 >> (8 * c));
                }
                bq[pp] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
              }
              grp[4 * d + c] = sk_mfma(xa, u32x4_v{bq[0], bq[1], bq[2], bq[3]}, Z ? zero : grp[4 * d + c]);
            }
          }
        }
      };
      // The group's scale, once per group (or at the end of the wave's steps):
      // tot += (grp - offset * rowsum(x)) * s, then the group sums start again from zero.
      auto fold = [&](const Slot& sl, auto zr) __attribute__((always_inline)) {
        float sc[CPL];
        const u32x4_v* ss = XT ? sw : sl.s;
        if constexpr (SF32) {
  #pragma unroll
          for (int c = 0; c < CPL; ++c) sc[c] = __uint_as_float(ss[c / 4][c % 4]);
        } else {
  #pragma unroll
          for (int c = 0; c < CPL; c += 2) {
            const uint32_t v = ss[c / 8][(c / 2) % 4];
            sc[c] = __uint_as_float(v << 16);
            sc[c + 1] = __uint_as_float(v & 0xFFFF0000u);
          }
        }
  #pragma unroll
        for (int c = 0; c < CPL; ++c)
  #pragma unroll
          for (int r = 0; r < MR; ++r)
            tot[c][r] = __builtin_fmaf(kOff != 0.0f ? grp[c][r] - kOff * sx[r] : grp[c][r], sc[c], tot[c][r]);
        if constexpr (decltype(zr)::value) {  // the next group's sums start from zero
  #pragma unroll
          for (int c = 0; c < CPL; ++c) grp[c] = zero;
          sx = zero;
        }
      };
      using False = std::integral_constant<bool, false>;
      using True = std::integral_constant<bool, true>;
      int crem = a.FS - k0 % a.FS;  // steps left in the current group, compute order
      // odd: the parity of t, known at each call site (slot A takes even steps, slot B odd ones).
      auto step = [&](const Slot& sl, int t, auto odd) __attribute__((always_inline)) {
        const u32x4_v& xa = kXW ? xw[kXW ? t : 0] : sl.x;
        if constexpr (G2) {
          // Even steps open a group, odd steps close it.
          if constexpr (!decltype(odd)::value) {
            compute(sl, xa, True{});
          } else {
            compute(sl, xa, False{});
            fold(sl, False{});
          }
        } else {
          compute(sl, xa, False{});
          if (--crem == 0 || t == a.T - 1) {
            fold(sl, True{});
            if (crem == 0) crem = a.FS;
          }
        }
      };
  
      if constexpr (XT == 4 && kXW) {
        // The same two-slot pipeline over exactly four steps, written out (static x indices).
        Slot A, B;
        issue(A, k0, False{});
        issue(B, k0 + 1, True{});
        __builtin_amdgcn_sched_barrier(0);
        step(A, 0, False{});
        __builtin_amdgcn_sched_barrier(0);
        issue(A, k0 + 2, False{});
        __builtin_amdgcn_sched_barrier(0);
        step(B, 1, True{});
        __builtin_amdgcn_sched_barrier(0);
        issue(B, k0 + 3, True{});
        __builtin_amdgcn_sched_barrier(0);
        step(A, 2, False{});
        step(B, 3, True{});
      } else if constexpr (PIPE) {
        // Two slots: step t + 2 is issued into a slot as soon as step t has used it, so each
        // wave keeps two steps of loads in flight while it computes.  The last two steps are
        // peeled off the loop so that every loop iteration issues the same loads.
        Slot A, B;
        issue(A, k0, False{});
        issue(B, k0 + 1, True{});
        __builtin_amdgcn_sched_barrier(0);
        int t = 0;
  #pragma unroll 1
        for (; t < a.T - 2; t += 2) {
          step(A, t, False{});
          __builtin_amdgcn_sched_barrier(0);
          issue(A, k0 + t + 2, False{});
          __builtin_amdgcn_sched_barrier(0);
          step(B, t + 1, True{});
          __builtin_amdgcn_sched_barrier(0);
          issue(B, k0 + t + 3, True{});
          __builtin_amdgcn_sched_barrier(0);
        }
        step(A, t, False{});
        step(B, t + 1, True{});
      } else {
        Slot A;
        issue(A, k0, False{});
        step(A, 0, False{});
      }
    }
  

  // Every wave's tile (rows < M) into LDS as [waves][M][kCols]; each output then adds the waves
  // in a fixed order.  Outputs are handled in quads (4 consecutive columns of one row).
  {
    float* rw = red + (size_t)wave * M * kCols;
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      const int row = 4 * kq + r;
      if (row < M) {
#pragma unroll
        for (int c = 0; c < CPL; c += 4)
          *(f32x4_t*)(rw + row * kCols + cg * CPL + c) = f32x4_t{tot[c][r], tot[c + 1][r], tot[c + 2][r], tot[c + 3][r]};
      }
    }
  }
  __syncthreads();
  if (mat + 1 < NM) {
#pragma unroll
    for (int i = 0; i < kMaxQ; ++i) {
      const int g = min(t + i * kThr, NQ - 1);
      *(f32x4_t*)(held + 4 * g) = wave_sum(g);
    }
    __syncthreads();  // the waves' tiles are free for the next product
  }
  }

  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      a.partial, (short)0, (int)((size_t)SP * M * a.N * sizeof(float)), 0x00020000);
  constexpr int kSc1 = 16;  // cache-policy operand of the buffer intrinsics: sc1
  if (a.S > 1) {
    // Split K: store this work item's tile of each product as [matrix][slice][M][N] (16-byte
    // stores with the agent-scope coherence bit sc1: visible across the XCDs' L2s without
    // whole-cache maintenance), wait until the stores have completed, then count the arrival.
    // Only the last arriver reads the tiles back, with loads that carry the same bit.
#pragma unroll
    for (int i = 0; i < kMaxQ; ++i) {
      const int g = t + i * kThr;
      const int m = g / kQPR, col = cblk + 4 * (g % kQPR);
      if (g < NQ && col < a.N) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_v, tile(0, i)), prs,
                                              (unsigned)(((slice * M + m) * a.N + col) * 4), 0, kSc1);
        if (a.pair)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_v, tile(1, i)), prs,
                                                (unsigned)((((a.S + slice) * M + m) * a.N + col) * 4), 0, kSc1);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(&a.counters[cb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev == (uint32_t)a.S - 1u;  // one arrival per slice
      if (last) __hip_atomic_store(&a.counters[cb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
  }

  // The outputs of the column block: the sum of the waves' tiles (one work item) or of the
  // partial tiles in slice order per matrix (each matrix's first tile taken as it is), then bias,
  // activation, bf16, and the folded elementwise op or the pair product, each rounded as the
  // separate ops round it, and one 8-byte store per quad.  The epilogue operands (bias, the pair's
  // second bias, the elementwise operand) are requested first, one vector load each, and the
  // partial tiles after them, so that all their latencies overlap; the plain case (bias at most)
  // takes a short path of its own, so that the activation code is not fetched.
  constexpr int kSl = 8;  // partial tiles per batch of loads (all in flight together)
  const bool plain = a.act == MX_ACT_NONE && !a.pair && !a.res_op;
#pragma unroll 1
  for (int i = 0; i < kMaxQ; ++i) {
    const int g = t + i * kThr;
    const int m = g / kQPR, col = cblk + 4 * (g % kQPR);
    if (g >= NQ || col >= a.N) continue;
    u32x4_v bq = {0u, 0u, 0u, 0u}, sq = bq;
    if (a.bias) bq = sk_quad_load(a.bias, col, a.b_dt);
    if (a.pair) {
      if (a.bias2) sq = sk_quad_load(a.bias2, col, a.b2_dt);
    } else if (a.res_op) {
      sq = sk_quad_load(a.res, (size_t)m * a.N + col, a.res_dt);
    }
    f32x4_t y, y2;
    if (a.S == 1) {
      // This workgroup holds every tile of the column block.
      y = tile(0, i);
      y2 = a.pair ? tile(1, i) : y;
    } else {
      y = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      y2 = y;
#pragma unroll 1
      for (int s0 = 0; s0 < SP; s0 += kSl) {
        f32x4_t v[kSl];
#pragma unroll
        for (int u = 0; u < kSl; ++u)
          v[u] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                 prs, (unsigned)(((min(s0 + u, SP - 1) * M + m) * a.N + col) * 4), 0, kSc1));
#pragma unroll
        for (int u = 0; u < kSl; ++u) {
          const int s = s0 + u;
          if (s < a.S)
            y = s == 0 ? v[u] : y + v[u];
          else if (s < SP)
            y2 = s == a.S ? v[u] : y2 + v[u];
        }
      }
    }
    const f32x4_t pre = a.bias ? y + sk_quad_value(bq, a.b_dt) : y;
    uint32_t o0, o1;
    if (plain) {
      o0 = (uint32_t)f32_to_bf16(pre[0]) | (uint32_t)f32_to_bf16(pre[1]) << 16;
      o1 = (uint32_t)f32_to_bf16(pre[2]) | (uint32_t)f32_to_bf16(pre[3]) << 16;
    } else {
      // The pair's second pre-activation value, or the elementwise operand.
      f32x4_t sec = y2;
      if (a.pair) {
        if (a.bias2) sec = y2 + sk_quad_value(sq, a.b2_dt);
      } else if (a.res_op) {
        sec = sk_quad_value(sq, a.res_dt);
      }
      o0 = 0u;
      o1 = 0u;
#pragma unroll 1
      for (int e = 0; e < 4; ++e) {
        const float pe = e == 0 ? pre[0] : e == 1 ? pre[1] : e == 2 ? pre[2] : pre[3];
        const float se = e == 0 ? sec[0] : e == 1 ? sec[1] : e == 2 ? sec[2] : sec[3];
        uint16_t v = f32_to_bf16(act_fast(pe, a.act));
        if (a.pair) {
          const uint16_t gv = f32_to_bf16(act_fast(se, a.act2));
          v = f32_to_bf16(mul_rn(bf16_to_f32(v), bf16_to_f32(gv)));
        } else if (a.res_op) {
          const float vf = bf16_to_f32(v);
          v = f32_to_bf16(a.res_op == MX_OP_MUL ? mul_rn(vf, se) : add_rn(vf, se));
        }
        const uint32_t sh = 16u * (uint32_t)(e & 1);
        if (e < 2)
          o0 |= (uint32_t)v << sh;
        else
          o1 |= (uint32_t)v << sh;
      }
    }
    *(u32x2_v*)(a.out + (size_t)m * a.N + col) = u32x2_v{o0, o1};
  }
}

// ---------------------------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------------------------
bool qdense_skinny_fits(const QDenseDesc& d) {
  const int64_t G = std::min<int64_t>(d.block_size, d.K);
  auto aligned = [](const void* p, size_t al) { return ((uintptr_t)p % al) == 0; };
  return d.M >= 1 && d.M <= kSkMaxRows && d.x_dt == MX_DTYPE_BFLOAT16 && d.scheme == MX_QUANT_LINEAR && !d.zp &&
         d.block_axis == 0 && d.K >= 32 && d.K % 32 == 0 && G % 32 == 0 && d.N >= 16 &&
         d.N % (dtype_is_packed(d.w_dt) ? 32 : 16) == 0 && d.K < (int64_t)1 << 30 && d.N < (int64_t)1 << 30 &&
         (d.s_dt == MX_DTYPE_BFLOAT16 || d.s_dt == MX_DTYPE_FLOAT32) && aligned(d.w, 16) && aligned(d.x, 16) &&
         aligned(d.scale, 16) && aligned(d.out, 8) && aligned(d.bias, 16) && aligned(d.res, 16) &&
         (!d.pair || (aligned(d.w2, 16) && aligned(d.scale2, 16) && aligned(d.bias2, 16) && d.res_op == 0));
}

// Steps per wave T: 1 when K/32 is odd; else the smallest even divisor of K/32 whose grid (column
// blocks x slices of `waves` wave-chunks) is within the resident workgroups (one per CU with 8
// waves, two with 4), so that the whole grid is resident at once (the largest even divisor when
// none is).  T and the wave count fix the summation order, so they depend on the shape of one
// product only: a pair launch sums each product exactly as its own launch would.
static int skinny_steps(const QDenseDesc& d, int64_t nb, int num_cus, int waves) {
  const int64_t ks = d.K / 32;
  if (ks % 2 != 0) return 1;
  int64_t best = 0;
  for (int64_t T = 2; T <= ks; T += 2) {
    if (ks % T != 0) continue;
    best = T;
    const int64_t S = (ks / T + waves - 1) / waves;
    if (nb * S <= (int64_t)num_cus * (kSkWaves / waves)) break;
  }
  return (int)best;
}

// Waves per workgroup: for one row when the 8-wave grid would fill at most three quarters of the
// CUs, 7 where seven waves of four steps (one scale group) give one workgroup per CU on at least
// three quarters of them (C2: 215 workgroups, at most 28 wave-steps per CU, 9.12 us against
// 9.25 us as 344 of 4, where 88 CUs took two workgroups), else 4 (C2 as 344 of 4: 9.7-9.9 us
// against 10.1-10.4 us as 172 of 8); 8 otherwise (batched shapes measured slower with 4: C3
// 18.1 -> 20.4 us, the MLP 41.5 -> 50.4 us).
static int skinny_waves(const QDenseDesc& d, int64_t nb, int num_cus) {
  if (d.M != 1) return kSkWaves;
  const int64_t T8 = skinny_steps(d, nb, num_cus, kSkWaves);
  const int64_t S8 = (d.K / 32 / T8 + kSkWaves - 1) / kSkWaves;
  if (4 * nb * S8 > 3 * (int64_t)num_cus) return kSkWaves;
  // Seven waves of four steps in one scale group, one workgroup per CU filling at least three
  // quarters of them.
  const int64_t T7 = skinny_steps(d, nb, num_cus, 7);
  const int64_t S7 = (d.K / 32 / T7 + 6) / 7;
  const int64_t G = std::min<int64_t>(d.block_size, d.K) / 32;
  if (T7 == 4 && G % 4 == 0 && nb * S7 <= num_cus && 4 * nb * S7 >= 3 * (int64_t)num_cus) return 7;
  return 4;
}

template <int WDT, int MR, bool SF32, int WV = kSkWaves>
static void launch_pipe(const SkinnyArgs& ga, int grid, size_t lds, hipStream_t st) {
  // Four steps per wave within one scale group (every wave's first step is a multiple of 4 and
  // FS % 4 == 0): the scales (and with one row, x) are loaded once per wave.
  if (ga.T == 4 && ga.FS % 4 == 0) {
    dispatch(qdense_skinny_kernel<WDT, MR, SF32, true, false, WV, 4>, grid, 64 * WV, lds, st, ga.x, ga.w, ga.scale, ga.K, ga.N, ga.T, ga.FS, ga.S, ga);
    return;
  }
  if (ga.T >= 2 && ga.FS == 2)
    dispatch(qdense_skinny_kernel<WDT, MR, SF32, true, true, WV>, grid, 64 * WV, lds, st, ga.x, ga.w, ga.scale, ga.K, ga.N, ga.T, ga.FS, ga.S, ga);
  else if (ga.T >= 2)
    dispatch(qdense_skinny_kernel<WDT, MR, SF32, true, false, WV>, grid, 64 * WV, lds, st, ga.x, ga.w, ga.scale, ga.K, ga.N, ga.T, ga.FS, ga.S, ga);
  else
    dispatch(qdense_skinny_kernel<WDT, MR, SF32, false, false, WV>, grid, 64 * WV, lds, st, ga.x, ga.w, ga.scale, ga.K, ga.N, ga.T, ga.FS, ga.S, ga);
}

template <int WDT>
static void launch_skinny(const SkinnyArgs& ga, bool sf32, int waves, int grid, size_t lds, hipStream_t st) {
  if (ga.M == 1 && waves == 7) {  // four steps per wave in one scale group (the plan checks)
    if (sf32)
      dispatch(qdense_skinny_kernel<WDT, 1, true, true, false, 7, 4>, grid, 64 * 7, lds, st, ga.x, ga.w, ga.scale, ga.K, ga.N, ga.T, ga.FS, ga.S, ga);
    else
      dispatch(qdense_skinny_kernel<WDT, 1, false, true, false, 7, 4>, grid, 64 * 7, lds, st, ga.x, ga.w, ga.scale, ga.K, ga.N, ga.T, ga.FS, ga.S, ga);
  } else if (ga.M == 1 && waves == 4) {
    if (sf32)
      launch_pipe<WDT, 1, true, 4>(ga, grid, lds, st);
    else
      launch_pipe<WDT, 1, false, 4>(ga, grid, lds, st);
  } else if (ga.M == 1) {
    if (sf32)
      launch_pipe<WDT, 1, true>(ga, grid, lds, st);
    else
      launch_pipe<WDT, 1, false>(ga, grid, lds, st);
  } else {
    if (sf32)
      launch_pipe<WDT, 4, true>(ga, grid, lds, st);
    else
      launch_pipe<WDT, 4, false>(ga, grid, lds, st);
  }
}

int qdense_skinny_run(mx_backend* b, const QDenseDesc& d, const char* name) {
  const bool i4 = dtype_is_packed(d.w_dt);
  const int64_t cols = i4 ? 256 : 128;
  const int64_t nb = (d.N + cols - 1) / cols;
  // The split (T, S, waves) fixes the summation order, so it is planned for MI355X's 256 CUs
  // whatever the device reports: the same inputs give the same bits on every device.
  const int ncu = kSkPlanCUs;
  const int waves = skinny_waves(d, nb, ncu);
  const int T = skinny_steps(d, nb, ncu, waves);
  const int64_t chunks = d.K / 32 / T;  // wave-sized pieces of one column block
  const int64_t S = (chunks + waves - 1) / waves;
  const int64_t SP = d.pair ? 2 * S : S;  // partial tiles per column block
  const size_t counter_bytes = 64 * 1024;
  if ((size_t)nb * 4 > counter_bytes || nb * SP > (int64_t)1 << 30 || SP * d.M * d.N * 4 >= (int64_t)1 << 31)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: N=%lld too large for the skinny path", (long long)d.N);
  SkinnyArgs ga;
  ga.x = (const uint16_t*)d.x;
  ga.w = (const uint8_t*)d.w;
  ga.scale = d.scale;
  ga.bias = d.bias;
  ga.out = (uint16_t*)d.out;
  ga.partial = nullptr;
  ga.counters = nullptr;
  if (SP > 1) {
    void* scratch = nullptr;
    MX_TRY(ensure_scratch(b, counter_bytes + (size_t)SP * d.M * d.N * sizeof(float), &scratch));
    ga.counters = (uint32_t*)scratch;
    ga.partial = (float*)((char*)scratch + counter_bytes);
  }
  ga.M = (int)d.M;
  ga.K = (int)d.K;
  ga.N = (int)d.N;
  ga.FS = (int)(std::min<int64_t>(d.block_size, d.K) / 32);
  ga.T = T;
  ga.S = (int)S;
  ga.act = d.act;
  ga.b_dt = d.b_dt;
  ga.res = d.res;
  ga.res_dt = d.res_dt;
  ga.res_op = d.res_op;
  ga.w2 = (const uint8_t*)d.w2;
  ga.scale2 = d.scale2;
  ga.bias2 = d.bias2;
  ga.pair = d.pair ? 1 : 0;
  ga.act2 = d.act2;
  ga.b2_dt = d.b2_dt;
  const int grid = (int)(nb * S);
  // LDS: the waves' tiles [waves][M][cols] and the first product's tile [M][cols].
  const size_t lds = (size_t)(waves + 1) * d.M * cols * sizeof(float);
  const bool sf32 = d.s_dt == MX_DTYPE_FLOAT32;
  hipStream_t st = b->stream;
  return launch(b, name, [&] {
    switch (d.w_dt) {
      case MX_DTYPE_INT4: launch_skinny<MX_DTYPE_INT4>(ga, sf32, waves, grid, lds, st); break;
      case MX_DTYPE_UINT4: launch_skinny<MX_DTYPE_UINT4>(ga, sf32, waves, grid, lds, st); break;
      case MX_DTYPE_INT8: launch_skinny<MX_DTYPE_INT8>(ga, sf32, waves, grid, lds, st); break;
      default: launch_skinny<MX_DTYPE_UINT8>(ga, sf32, waves, grid, lds, st); break;
    }
  });
}

}  // namespace mx
