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
// The kernel is HBM-bound: every weight byte is read once.  Weights stream from HBM straight
// into LDS with direct global->LDS loads (16 bytes per lane, no registers involved), so each
// wave keeps several K steps in flight in a private LDS ring; a step is then read from LDS and
// dequantised in registers into the B operand of v_mfma_f32_16x16x32_bf16 (the matrix cores do
// the multiply-adds, the VALU only converts).  The 16 rows of the MFMA A operand are the rows of
// x (rows >= M repeat row M-1 and are never stored).
//
// Lane layout (wave of 64 lanes, cg = lane % 16, kq = lane / 16; CPL = columns per lane, 4, 8 or
// 16, so a workgroup covers 16*CPL columns).  In one 32-row K step a lane uses rows
// k0 + 8*kq + e (e = 0..7) of its CPL consecutive columns col0 = CPL*cg.  MFMA number c takes
// column col0 + c from every lane, so its result column j = cg is block column CPL*j + c, and the
// lane ends up holding rows 4*kq + r (r = 0..3) of its own CPL columns.
//
// Dequantisation into bf16 pairs (two K rows of one column per dword):
//   int8/uint8: exact conversion through f32 (|w| < 256 has at most 8 significant bits), the
//               two high halves packed with one v_perm;
//   int4/uint4: v_perm gathers the bytes of two rows, then and/xor turn a nibble u into the
//               bf16 bit pattern 0x4300|u = 128 + u (exact); for Int4 the xor also flips bit 3,
//               giving 136 + w.  The offset is removed per group with the group's row sums of
//               x, which one extra MFMA against an all-ones B operand produces.
//
// Work decomposition.  A workgroup (NW = 16, 8 or 4 waves for CPL = 4, 8, 16) owns 16*CPL output
// columns and one of S slices of the K steps; its waves split the slice's steps.  The host picks
// CPL and S so that about one workgroup per CU covers the matrix, preferring S = 1 (no split-K)
// and then narrow column blocks over more slices.  The waves' partial tiles are summed through LDS; with S > 1 every
// workgroup stores its tile to scratch and the last one to arrive for the column block adds the
// S tiles in slice order (deterministic), adds the bias, applies the activation and rounds to
// bf16.
#include <algorithm>
#include <cmath>

#include "device_common.h"
#include "mxrt_internal.h"

namespace mx {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef __attribute__((address_space(1))) void* gbl_void_ptr;

constexpr int kSkMaxRows = 16;
constexpr int kSkRingBytes = 144 * 1024;  // LDS rings of a workgroup (one workgroup per CU)

struct SkinnyArgs {
  const uint16_t* x;    // [M, K] bf16
  const uint8_t* w;     // [K, N] storage bytes
  const void* scale;    // [ceil(K/G), N]
  const void* bias;     // [N] or null
  uint16_t* out;        // [M, N] bf16
  float* partial;       // [S, M, N] (S > 1)
  uint32_t* counters;   // [column blocks]
  int M, K, N, G, S, act, b_dt;
};

// Geometry of one instantiation: CPL columns per lane, NW waves per workgroup.  Narrow blocks
// take more waves, so that each CU has enough waves to overlap one wave's step latency (DMA
// wait, LDS reads, conversion, MFMA, group flush) with the others' work.
template <int WDT, int CPL, int NW>
struct SkGeom {
  static constexpr bool kI4 = WDT == MX_DTYPE_INT4 || WDT == MX_DTYPE_UINT4;
  static constexpr int kCols = 16 * CPL;                     // columns per workgroup
  static constexpr int kRowBytes = kI4 ? kCols / 2 : kCols;  // bytes of one K row of the block
  static constexpr int kLaneBytes = kRowBytes / 16;          // bytes per lane per row (4/8/16)
  static constexpr int kWBytes = 32 * kRowBytes;             // weight bytes per 32-row step
  static constexpr int kWInstr = kWBytes / 1024;             // 16-byte-per-lane DMA loads
  static constexpr int kSlot = kWBytes + 2048;               // + x block (1 KB) + scales (1 KB)
  static constexpr int kD0 = kSkRingBytes / (NW * kSlot);
  static constexpr int kD = kD0 > 7 ? 7 : kD0;               // steps in flight per wave
  static constexpr int kP = kWInstr + 2;                     // DMA instructions per step
  static constexpr int kRing = NW * kD * kSlot;              // LDS of the workgroup's rings
  static constexpr int kThreads = 64 * NW;
  static_assert(kLaneBytes == 4 || kLaneBytes == 8 || kLaneBytes == 16, "lane width");
  static_assert(kD >= 2 && kD <= 7 && (kD - 1) * kP < 64, "ring depth");
};

__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

__device__ __forceinline__ f32x4_t mfma16x16x32(const uint32_t (&a)[4], const uint32_t (&b)[4], f32x4_t c) {
  const u32x4_v av = {a[0], a[1], a[2], a[3]};
  const u32x4_v bv = {b[0], b[1], b[2], b[3]};
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), __builtin_bit_cast(bf16x8_t, bv),
                                                 c, 0, 0, 0);
}

// Workgroup index -> work item, so that the S slices of one column block (consecutive items)
// run on one XCD and share its L2: workgroups are dispatched round-robin over the 8 XCDs.
__device__ __forceinline__ int sk_xcd_swizzle(int bid, int total) {
  if ((total & 7) != 0) return bid;
  return (bid & 7) * (total >> 3) + (bid >> 3);
}

// Split-K completion for the partial tiles in scratch.  Every access to the shared partials is
// an agent-scope atomic (coherent across the XCDs' L2s without whole-cache maintenance); the
// s_waitcnt makes this workgroup's partial stores complete before its arrival is counted, and
// only the last arriver reads them back.  Returns true in every thread of the last arriver.
__device__ __forceinline__ bool sk_last_arriver(uint32_t* counter, uint32_t arrivals, int* s_flag) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == arrivals - 1u;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = last;
  }
  __syncthreads();
  return *s_flag != 0;
}

// One wave-wide direct load of 16 bytes per lane from global memory into LDS: lane L's bytes land
// at lds + 16*L (the LDS address must be the same in every lane).  The data does not pass
// through registers; completion is tracked by the wave's vmcnt like any vector load.
__device__ __forceinline__ void dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds((gbl_void_ptr)const_cast<void*>(src), (lds_void_ptr)lds, 16, 0, 0);
}

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt and lgkmcnt not waited for).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Byte address of an LDS location (the value a ds_read takes).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// LDS reads of one step's operands: 8 rows of this lane's weight bytes (row pitch 16*W) and its
// 16 bytes of x, issued back to back and completed together.  They are one asm block because
// the compiler, seeing ordinary LDS reads after LDS-DMA loads, would wait for every outstanding
// DMA (vmcnt(0)) before them and serialise the ring; the DMA into the slot is known complete
// from the caller's explicit vmcnt wait.
template <int W>
__device__ __forceinline__ void lds_read_step(uint32_t wa, uint32_t xa, uint32_t (&r)[8][W / 4], u32x4_v& x);

template <>
__device__ __forceinline__ void lds_read_step<4>(uint32_t wa, uint32_t xa, uint32_t (&r)[8][1], u32x4_v& x) {
  asm volatile(
      "ds_read_b32 %0, %9 offset:0\n\t"
      "ds_read_b32 %1, %9 offset:64\n\t"
      "ds_read_b32 %2, %9 offset:128\n\t"
      "ds_read_b32 %3, %9 offset:192\n\t"
      "ds_read_b32 %4, %9 offset:256\n\t"
      "ds_read_b32 %5, %9 offset:320\n\t"
      "ds_read_b32 %6, %9 offset:384\n\t"
      "ds_read_b32 %7, %9 offset:448\n\t"
      "ds_read_b128 %8, %10 offset:0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0][0]), "=&v"(r[1][0]), "=&v"(r[2][0]), "=&v"(r[3][0]), "=&v"(r[4][0]), "=&v"(r[5][0]),
        "=&v"(r[6][0]), "=&v"(r[7][0]), "=&v"(x)
      : "v"(wa), "v"(xa)
      : "memory");
}

template <>
__device__ __forceinline__ void lds_read_step<8>(uint32_t wa, uint32_t xa, uint32_t (&r)[8][2], u32x4_v& x) {
  u32x2_v q[8];
  asm volatile(
      "ds_read_b64 %0, %9 offset:0\n\t"
      "ds_read_b64 %1, %9 offset:128\n\t"
      "ds_read_b64 %2, %9 offset:256\n\t"
      "ds_read_b64 %3, %9 offset:384\n\t"
      "ds_read_b64 %4, %9 offset:512\n\t"
      "ds_read_b64 %5, %9 offset:640\n\t"
      "ds_read_b64 %6, %9 offset:768\n\t"
      "ds_read_b64 %7, %9 offset:896\n\t"
      "ds_read_b128 %8, %10 offset:0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3]), "=&v"(q[4]), "=&v"(q[5]), "=&v"(q[6]), "=&v"(q[7]),
        "=&v"(x)
      : "v"(wa), "v"(xa)
      : "memory");
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    r[e][0] = q[e].x;
    r[e][1] = q[e].y;
  }
}

template <>
__device__ __forceinline__ void lds_read_step<16>(uint32_t wa, uint32_t xa, uint32_t (&r)[8][4], u32x4_v& x) {
  u32x4_v q[8];
  asm volatile(
      "ds_read_b128 %0, %9 offset:0\n\t"
      "ds_read_b128 %1, %9 offset:256\n\t"
      "ds_read_b128 %2, %9 offset:512\n\t"
      "ds_read_b128 %3, %9 offset:768\n\t"
      "ds_read_b128 %4, %9 offset:1024\n\t"
      "ds_read_b128 %5, %9 offset:1280\n\t"
      "ds_read_b128 %6, %9 offset:1536\n\t"
      "ds_read_b128 %7, %9 offset:1792\n\t"
      "ds_read_b128 %8, %10 offset:0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3]), "=&v"(q[4]), "=&v"(q[5]), "=&v"(q[6]), "=&v"(q[7]),
        "=&v"(x)
      : "v"(wa), "v"(xa)
      : "memory");
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    r[e][0] = q[e].x;
    r[e][1] = q[e].y;
    r[e][2] = q[e].z;
    r[e][3] = q[e].w;
  }
}

// The scale bytes of this lane's columns (NB = 8, 16, 32 or 64 bytes) from LDS.
template <int NB>
__device__ __forceinline__ void lds_read_scales(uint32_t sa, uint32_t (&s)[NB / 4]) {
  if constexpr (NB == 8) {
    u32x2_v v;
    asm volatile("ds_read_b64 %0, %1 offset:0\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(sa) : "memory");
    s[0] = v.x;
    s[1] = v.y;
  } else {
    u32x4_v q[NB / 16];
    if constexpr (NB == 16) {
      asm volatile("ds_read_b128 %0, %1 offset:0\n\ts_waitcnt lgkmcnt(0)" : "=&v"(q[0]) : "v"(sa) : "memory");
    } else if constexpr (NB == 32) {
      asm volatile("ds_read_b128 %0, %2 offset:0\n\tds_read_b128 %1, %2 offset:16\n\ts_waitcnt lgkmcnt(0)"
                   : "=&v"(q[0]), "=&v"(q[1])
                   : "v"(sa)
                   : "memory");
    } else {
      asm volatile(
          "ds_read_b128 %0, %4 offset:0\n\tds_read_b128 %1, %4 offset:16\n\t"
          "ds_read_b128 %2, %4 offset:32\n\tds_read_b128 %3, %4 offset:48\n\ts_waitcnt lgkmcnt(0)"
          : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3])
          : "v"(sa)
          : "memory");
    }
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      s[4 * i] = q[i].x;
      s[4 * i + 1] = q[i].y;
      s[4 * i + 2] = q[i].z;
      s[4 * i + 3] = q[i].w;
    }
  }
}

// Waves per workgroup for a lane width.
template <int CPL>
constexpr int sk_waves() {
  return CPL == 4 ? 16 : (CPL == 8 ? 8 : 4);
}

template <int WDT, int SDT, int CPL, int NW>
__global__ __launch_bounds__(64 * NW) void qdense_skinny_kernel(SkinnyArgs a) {
  using Gm = SkGeom<WDT, CPL, NW>;
  constexpr bool kI4 = Gm::kI4;
  constexpr float kOff = WDT == MX_DTYPE_INT4 ? 136.0f : (WDT == MX_DTYPE_UINT4 ? 128.0f : 0.0f);
  constexpr uint32_t kNibXor = WDT == MX_DTYPE_INT4 ? 0x43084308u : 0x43004300u;
  constexpr int kSB = SDT == MX_DTYPE_BFLOAT16 ? 2 : 4;  // scale bytes
  constexpr int kD = Gm::kD;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_last;

  const int item = sk_xcd_swizzle(blockIdx.x, gridDim.x);
  const int cb = item / a.S, slice = item % a.S;
  // The wave index is wave-uniform; saying so keeps the K loop's control flow scalar.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int cg = lane & 15, kq = lane >> 4;
  const int T = a.K >> 5;
  const int sb = (int)((int64_t)slice * T / a.S), se = (int)((int64_t)(slice + 1) * T / a.S);
  const int wb = sb + wave * (se - sb) / NW, we = sb + (wave + 1) * (se - sb) / NW;
  uint8_t* ring = smem + (size_t)wave * kD * Gm::kSlot;
  const int cblk = cb * Gm::kCols;

  // DMA source addresses of this lane.  Chunks past the last column read column 0 instead
  // (their results are never stored), so no load needs a predicate.
  const size_t row_bytes = kI4 ? (size_t)(a.N >> 1) : (size_t)a.N;
  const size_t blk_bytes = kI4 ? (size_t)(cblk >> 1) : (size_t)cblk;
  const uint8_t* wsrc[Gm::kWInstr];
#pragma unroll
  for (int i = 0; i < Gm::kWInstr; ++i) {
    const int f = i * 1024 + lane * 16;  // byte of the step's row-major [32][kRowBytes] tile
    const int r = f / Gm::kRowBytes, ch = f % Gm::kRowBytes;
    const size_t cbyte = blk_bytes + ch + 16 <= row_bytes ? blk_bytes + ch : 0;
    wsrc[i] = a.w + (size_t)r * row_bytes + cbyte;
  }
  const uint16_t* xsrc = a.x + (size_t)min(lane & 15, a.M - 1) * a.K + 8 * (lane >> 4);
  const size_t s_row = (size_t)a.N * kSB;
  const size_t s_byte = (size_t)cblk * kSB + lane * 16;
  const char* ssrc = (const char*)a.scale + (s_byte + 16 <= s_row ? s_byte : 0);

  auto issue = [&](int j, uint8_t* slot) {
    const size_t step = (size_t)(32 * j) * row_bytes;
#pragma unroll
    for (int i = 0; i < Gm::kWInstr; ++i) dma16(wsrc[i] + step, slot + i * 1024);
    dma16(xsrc + 32 * j, slot + Gm::kWBytes);
    dma16(ssrc + (size_t)((32 * j) / a.G) * s_row, slot + Gm::kWBytes + 1024);
  };

  f32x4_t tot[CPL], grp[CPL], sx;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    tot[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    grp[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  sx = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Lane offsets of the LDS reads inside a slot.
  const uint32_t w_off = (uint32_t)(8 * kq * Gm::kRowBytes + cg * Gm::kLaneBytes);
  const uint32_t x_off = (uint32_t)(Gm::kWBytes + lane * 16);
  const uint32_t s_off = (uint32_t)(Gm::kWBytes + 1024 + cg * CPL * kSB);

  auto compute_step = [&](int j, const uint8_t* slot) {
    // The group's sums are folded into the totals after its last step (or after the wave's last
    // step when the wave's range ends inside a group).
    const bool flush = (j + 1 == we) || ((32 * (j + 1)) % a.G == 0);
    const uint32_t sbase = lds_addr(slot);
    uint32_t r[8][Gm::kLaneBytes / 4], xv[4];
    {
      u32x4_v xq;
      lds_read_step<Gm::kLaneBytes>(sbase + w_off, sbase + x_off, r, xq);
      xv[0] = xq.x;
      xv[1] = xq.y;
      xv[2] = xq.z;
      xv[3] = xq.w;
    }
    if constexpr (kI4) {
#pragma unroll
      for (int d = 0; d < CPL / 8; ++d) {
        uint32_t bq[8][4];  // columns 8d + 0..7, four pair-dwords each
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const uint32_t A = r[2 * pp][d], B = r[2 * pp + 1][d];
          const uint32_t t0 = __builtin_amdgcn_perm(B, A, 0x06040200u);  // [A.b0, A.b2, B.b0, B.b2]
          const uint32_t t1 = __builtin_amdgcn_perm(B, A, 0x07050301u);  // [A.b1, A.b3, B.b1, B.b3]
          bq[0][pp] = ((t0 >> 0) & 0x000F000Fu) ^ kNibXor;
          bq[1][pp] = ((t0 >> 4) & 0x000F000Fu) ^ kNibXor;
          bq[4][pp] = ((t0 >> 8) & 0x000F000Fu) ^ kNibXor;
          bq[5][pp] = ((t0 >> 12) & 0x000F000Fu) ^ kNibXor;
          bq[2][pp] = ((t1 >> 0) & 0x000F000Fu) ^ kNibXor;
          bq[3][pp] = ((t1 >> 4) & 0x000F000Fu) ^ kNibXor;
          bq[6][pp] = ((t1 >> 8) & 0x000F000Fu) ^ kNibXor;
          bq[7][pp] = ((t1 >> 12) & 0x000F000Fu) ^ kNibXor;
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) grp[8 * d + c] = mfma16x16x32(xv, bq[c], grp[8 * d + c]);
      }
      const uint32_t ones[4] = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
      sx = mfma16x16x32(xv, ones, sx);
    } else {
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int dw = c >> 2, sh = 8 * (c & 3);
        uint32_t bq[4];
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          float f0, f1;
          if constexpr (WDT == MX_DTYPE_INT8) {
            f0 = (float)(int8_t)(r[2 * pp][dw] >> sh);
            f1 = (float)(int8_t)(r[2 * pp + 1][dw] >> sh);
          } else {
            f0 = (float)(uint8_t)(r[2 * pp][dw] >> sh);
            f1 = (float)(uint8_t)(r[2 * pp + 1][dw] >> sh);
          }
          bq[pp] = pack_hi16(f0, f1);
        }
        grp[c] = mfma16x16x32(xv, bq, grp[c]);
      }
    }
    if (flush) {
      uint32_t sv[CPL * kSB / 4];
      lds_read_scales<CPL * kSB>(sbase + s_off, sv);
      float sc[CPL];
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        if constexpr (SDT == MX_DTYPE_BFLOAT16)
          sc[c] = __uint_as_float((c & 1) ? (sv[c >> 1] & 0xFFFF0000u) : (sv[c >> 1] << 16));
        else
          sc[c] = __uint_as_float(sv[c]);
      }
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float v = kOff != 0.0f ? grp[c][q] - kOff * sx[q] : grp[c][q];
          tot[c][q] += v * sc[c];
        }
        grp[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
      sx = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  };

  // Pipeline: kD steps in flight per wave.  Step j's DMA has completed once at most
  // (number of steps issued after it) * kP vector-memory instructions are outstanding; its
  // slot is refilled with step j + kD after it has been read.
  for (int d = 0; d < kD; ++d)
    if (wb + d < we) issue(wb + d, ring + d * Gm::kSlot);
  for (int j = wb; j < we; ++j) {
    uint8_t* slot = ring + ((j - wb) % kD) * Gm::kSlot;
    const int newer = min(kD - 1, we - 1 - j);
    switch (newer) {  // ring tail: fewer steps were issued after this one
      case 0: wait_vmcnt<0>(); break;
      case 1: wait_vmcnt<Gm::kP>(); break;
      case 2: wait_vmcnt<(kD > 2 ? 2 : 0) * Gm::kP>(); break;
      case 3: wait_vmcnt<(kD > 3 ? 3 : 0) * Gm::kP>(); break;
      case 4: wait_vmcnt<(kD > 4 ? 4 : 0) * Gm::kP>(); break;
      case 5: wait_vmcnt<(kD > 5 ? 5 : 0) * Gm::kP>(); break;
      default: wait_vmcnt<(kD > 6 ? 6 : 0) * Gm::kP>(); break;
    }
    compute_step(j, slot);  // its LDS reads have completed (lgkmcnt(0) inside)
    if (j + kD < we) issue(j + kD, slot);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // the rings are reused below

  // Every wave's tile (rows < M) into LDS as [NW waves][M][cols] (the rings' memory); then the
  // block's M x cols outputs are shared out over the threads, each adding the waves in a fixed
  // order.  A thread's outputs all lie in one column (the thread count is a multiple of the
  // block width), so its bias is loaded once.
  constexpr int kC = Gm::kCols;
  float* red = (float*)smem;
  const int M = a.M;
  {
    float* rw = red + (size_t)wave * M * kC;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = 4 * kq + q;
      if (row < M) {
#pragma unroll
        for (int c = 0; c < CPL; c += 4)
          *(float4*)(rw + row * kC + cg * CPL + c) = make_float4(tot[c][q], tot[c + 1][q], tot[c + 2][q], tot[c + 3][q]);
      }
    }
  }
  __syncthreads();
  constexpr int kThreads = Gm::kThreads;
  static_assert(kThreads % kC == 0, "one column per thread");
  const int t = threadIdx.x;
  const int MC = M * kC;
  const int n_t = cblk + t % kC;
  const float bias_t = (a.bias && n_t < a.N) ? load_f(a.bias, n_t, a.b_dt) : 0.0f;
  auto finish = [&](int p, float y) {
    const int m = p / kC;
    if (n_t < a.N) a.out[(size_t)m * a.N + n_t] = f32_to_bf16(act_fast(y + bias_t, a.act));
  };
  auto wave_sum = [&](int p) {
    float v = red[p];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += red[w * MC + p];
    return v;
  };
  if (a.S == 1) {
    for (int p = t; p < MC; p += kThreads) finish(p, wave_sum(p));
    return;
  }
  for (int p = t; p < MC; p += kThreads) {
    const int m = p / kC, n = cblk + p % kC;
    if (n < a.N)
      __hip_atomic_store(&a.partial[((size_t)slice * M + m) * a.N + n], wave_sum(p), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!sk_last_arriver(&a.counters[cb], (uint32_t)a.S, &s_last)) return;
  // Last arriver: each output adds the S slices in slice order, 8 loads in flight at a time.
  for (int p = t; p < MC; p += kThreads) {
    const int m = p / kC;
    const int n = min(n_t, a.N - 1);
    const float* src = a.partial + (size_t)m * a.N + n;
    const size_t ss = (size_t)M * a.N;
    float y = 0.0f;
    for (int s0 = 0; s0 < a.S; s0 += 8) {
      float pv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        pv[u] = __hip_atomic_load(src + (size_t)min(s0 + u, a.S - 1) * ss, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int u = 0; u < 8; ++u) y += s0 + u < a.S ? pv[u] : 0.0f;
    }
    finish(p, y);
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
         aligned(d.w, 16) && aligned(d.x, 16) && aligned(d.scale, 16);
}

// Columns per lane and number of K slices.  Each option covers the columns with 16*CPL-wide
// blocks and takes S = floor(CUs / blocks) slices (at least 1), so about one workgroup per CU
// (the rings take most of a CU's LDS).  The best option fills the most CUs in its last round;
// ties go to fewer slices (no split-K is best: no partials, no completion protocol), then to
// wider blocks.
struct SkPlan {
  int cpl = 16, S = 1;
};

static SkPlan skinny_plan(const QDenseDesc& d, int num_cus) {
  const bool i4 = dtype_is_packed(d.w_dt);
  const int64_t cus = std::max(num_cus, 1);
  const int64_t steps = d.K / 32;
  SkPlan best;
  double best_u = -1.0;
  for (int cpl : {16, 8, 4}) {
    if (i4 && cpl == 4) continue;
    const int64_t nb = (d.N + 16 * cpl - 1) / (16 * cpl);
    int64_t S = std::max<int64_t>(1, cus / nb);
    const int nw = cpl == 4 ? 16 : (cpl == 8 ? 8 : 4);
    S = std::min<int64_t>(S, std::max<int64_t>(1, steps / (2 * nw)));  // each wave keeps >= 2 steps
    S = std::min<int64_t>(S, std::max<int64_t>(1, 120 / d.M));
    const int64_t wgs = nb * S;
    const int64_t rounds = (wgs + cus - 1) / cus;
    const double u = (double)wgs / (double)(rounds * cus);
    if (u > best_u + 1e-9 || (std::fabs(u - best_u) <= 1e-9 && S < best.S)) {
      best_u = u;
      best.cpl = cpl;
      best.S = (int)S;
    }
  }
  return best;
}

template <int WDT, int SDT, int CPL>
static void launch_one(const SkinnyArgs& ga, int grid, hipStream_t st) {
  constexpr int NW = sk_waves<CPL>();
  using Gm = SkGeom<WDT, CPL, NW>;
  // The rings; after the K loop the same memory holds the waves' tiles (NW x M rows).
  const size_t lds = std::max<size_t>(Gm::kRing, (size_t)NW * ga.M * Gm::kCols * sizeof(float));
  qdense_skinny_kernel<WDT, SDT, CPL, NW><<<grid, Gm::kThreads, lds, st>>>(ga);
}

template <int WDT, int SDT>
static void launch_cpl(const SkinnyArgs& ga, int cpl, int grid, hipStream_t st) {
  if (cpl == 16) {
    launch_one<WDT, SDT, 16>(ga, grid, st);
  } else if (cpl == 8) {
    launch_one<WDT, SDT, 8>(ga, grid, st);
  } else {
    if constexpr (WDT == MX_DTYPE_INT8 || WDT == MX_DTYPE_UINT8) launch_one<WDT, SDT, 4>(ga, grid, st);
  }
}

template <int WDT>
static void launch_skinny(const SkinnyArgs& ga, int cpl, int grid, int sdt, hipStream_t st) {
  if (sdt == MX_DTYPE_BFLOAT16)
    launch_cpl<WDT, MX_DTYPE_BFLOAT16>(ga, cpl, grid, st);
  else
    launch_cpl<WDT, MX_DTYPE_FLOAT32>(ga, cpl, grid, st);
}

int qdense_skinny_run(mx_backend* b, const QDenseDesc& d, const char* name) {
  const SkPlan plan = skinny_plan(d, b->num_cus);
  const int64_t nb = (d.N + 16 * plan.cpl - 1) / (16 * plan.cpl);
  const int S = plan.S;
  const size_t counter_bytes = 64 * 1024;
  if ((size_t)nb * 4 > counter_bytes || nb * S > (int64_t)1 << 30)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: N=%lld too large for the skinny path", (long long)d.N);
  SkinnyArgs ga;
  ga.x = (const uint16_t*)d.x;
  ga.w = (const uint8_t*)d.w;
  ga.scale = d.scale;
  ga.bias = d.bias;
  ga.out = (uint16_t*)d.out;
  ga.partial = nullptr;
  ga.counters = nullptr;
  if (S > 1) {
    void* scratch = nullptr;
    MX_TRY(ensure_scratch(b, counter_bytes + (size_t)S * d.M * d.N * sizeof(float), &scratch));
    ga.counters = (uint32_t*)scratch;
    ga.partial = (float*)((char*)scratch + counter_bytes);
  }
  ga.M = (int)d.M;
  ga.K = (int)d.K;
  ga.N = (int)d.N;
  ga.G = (int)std::min<int64_t>(d.block_size, d.K);
  ga.S = S;
  ga.act = d.act;
  ga.b_dt = d.b_dt;
  const int grid = (int)(nb * S);
  hipStream_t st = b->stream;
  return launch(b, name, [&] {
    switch (d.w_dt) {
      case MX_DTYPE_INT4: launch_skinny<MX_DTYPE_INT4>(ga, plan.cpl, grid, d.s_dt, st); break;
      case MX_DTYPE_UINT4: launch_skinny<MX_DTYPE_UINT4>(ga, plan.cpl, grid, d.s_dt, st); break;
      case MX_DTYPE_INT8: launch_skinny<MX_DTYPE_INT8>(ga, plan.cpl, grid, d.s_dt, st); break;
      default: launch_skinny<MX_DTYPE_UINT8>(ga, plan.cpl, grid, d.s_dt, st); break;
    }
  });
}

}  // namespace mx
