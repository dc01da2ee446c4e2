// Prefill FusedQuantizedDense on gfx950: a bf16 MFMA GEMM with the int8 weights dequantised on
// the fly, for M > 16 rows of bf16 activations and one scale per output column.
//
// Reference semantics: quantizedDenseLinearInt (internal/gobackend/fusedops/quantizeddense.go:
// 616-650) then the activation epilogue (fusedops/dense.go:176-205).  With a per-channel scale
// s[n] the reference's terms (x*w)*s factor as  y[m,n] = act(bias[n] + s[n] * sum_k x[m,k]*w[k,n]);
// every product x*w is exact in f32, so only the summation order differs from the reference.
//
// Tiling.  A workgroup (8 waves, two per SIMD) computes a 256 x 128 output tile; wave w owns
// rows [64 wr, 64 wr + 64) x columns [64 wc, 64 wc + 64) with wr = w % 4, wc = w / 4.  K advances
// in blocks of 64 through a 3-stage LDS ring filled by direct global->LDS loads (16 bytes per
// lane, issued two blocks ahead):
//   - x tile [256 rows][64 k] bf16 (32 KB), its 16-byte chunks XOR-swizzled within each row by
//     (row >> 1) & 7 so that the 16 rows of an MFMA operand read land in distinct LDS banks;
//   - w tile [64 k][128 columns] int8 (8 KB), stored as 8 blocks of 8 rows with a 64-byte gap
//     between blocks so that the four row groups read together use different banks.
// Per 32-row K step a wave reads its 4 row blocks of x as the A operands of
// v_mfma_f32_16x16x32_bf16 and, for B, 8 rows x 4 columns of int8 per lane, converted exactly to
// bf16 pairs (|w| < 256 has at most 8 significant bits) in registers: 4 B operands (column c of
// every lane's 4 columns), 16 MFMAs per step.  With two waves per SIMD one wave's conversion
// overlaps the other's MFMAs.  Lane (cg = lane % 16, kq = lane / 16) ends with rows 4*kq + r of
// each 16-row block and the 4 consecutive columns 4*cg .. 4*cg + 3 of its wave's 64; the
// epilogue applies scale, bias and activation and writes 8-byte bf16 runs.
// Tile order: every XCD (workgroups are dispatched round-robin over the 8) takes a 2 x 16 block
// of tiles, so its L2 serves the x rows and w columns they share.
#include <algorithm>

#include "device_common.h"
#include "mxrt_internal.h"

namespace mx {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef __attribute__((address_space(1))) void* gbl_void_ptr;

constexpr int kBM = 256, kBN = 128, kBK = 64, kWaves = 8, kThreads = 64 * kWaves, kStages = 3;
constexpr int kABytes = kBM * kBK * 2;              // 32 KB
constexpr int kBPitch = 8 * kBN + 64;               // one 8-row block of w plus the bank gap
constexpr int kBBytes = (kBK / 8) * kBPitch;        // 8.5 KB
constexpr int kStage = kABytes + kBBytes;
constexpr int kLds = kStages * kStage;
constexpr int kAInstr = kABytes / (kWaves * 1024);  // DMA loads per wave per stage (x)
constexpr int kBInstr = (kBK / 8) / kWaves;         // DMA loads per wave per stage (w)
constexpr int kP = kAInstr + kBInstr;
static_assert(kAInstr * kWaves * 1024 == kABytes && kBInstr * kWaves == kBK / 8, "DMA split");

struct GemmArgs {
  const uint16_t* x;  // [M, K] bf16
  const uint8_t* w;   // [K, N] int8 / uint8
  const void* scale;  // [N]
  const void* bias;   // [N] or null
  uint16_t* out;      // [M, N] bf16
  int M, K, N, s_dt, b_dt, act, tiles_n, grouped;
};

__device__ __forceinline__ void dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds((gbl_void_ptr)const_cast<void*>(src), (lds_void_ptr)lds, 16, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__device__ __forceinline__ f32x4_t mfma(const u32x4_v& a, const u32x4_v& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

// One K step's operands from LDS: the wave's 4 x-row blocks (16 bytes each, blocks 2 KB apart)
// and 8 rows x 4 bytes of w.  One asm block completes them together: ordinary LDS reads after
// LDS-DMA loads would make the compiler wait for every outstanding DMA.
__device__ __forceinline__ void read_step(uint32_t aa, uint32_t ba, u32x4_v (&A)[4], uint32_t (&B)[8]) {
  asm volatile(
      "ds_read_b128 %0, %12 offset:0\n\t"
      "ds_read_b128 %1, %12 offset:2048\n\t"
      "ds_read_b128 %2, %12 offset:4096\n\t"
      "ds_read_b128 %3, %12 offset:6144\n\t"
      "ds_read_b32 %4, %13 offset:0\n\t"
      "ds_read_b32 %5, %13 offset:128\n\t"
      "ds_read_b32 %6, %13 offset:256\n\t"
      "ds_read_b32 %7, %13 offset:384\n\t"
      "ds_read_b32 %8, %13 offset:512\n\t"
      "ds_read_b32 %9, %13 offset:640\n\t"
      "ds_read_b32 %10, %13 offset:768\n\t"
      "ds_read_b32 %11, %13 offset:896\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(A[0]), "=&v"(A[1]), "=&v"(A[2]), "=&v"(A[3]), "=&v"(B[0]), "=&v"(B[1]), "=&v"(B[2]), "=&v"(B[3]),
        "=&v"(B[4]), "=&v"(B[5]), "=&v"(B[6]), "=&v"(B[7])
      : "v"(aa), "v"(ba)
      : "memory");
}

// Four outputs of one row: scale, bias, activation, bf16.  Kept out of line: inlined at all 16
// call sites of the epilogue the activation code would be tens of KB of instructions.
struct F4 {
  float v[4];
};
__device__ __attribute__((noinline)) uint2 epilogue4(F4 y, F4 sc, F4 bi, int act) {
  uint32_t o[2];
#pragma unroll
  for (int c = 0; c < 4; c += 2) {
    const uint32_t lo = f32_to_bf16(act_fast(y.v[c] * sc.v[c] + bi.v[c], act));
    const uint32_t hi = f32_to_bf16(act_fast(y.v[c + 1] * sc.v[c + 1] + bi.v[c + 1], act));
    o[c / 2] = lo | (hi << 16);
  }
  return make_uint2(o[0], o[1]);
}

template <int WDT>
__global__ __launch_bounds__(kThreads) void qdense_gemm_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  // Tile order: consecutive work items go to one XCD (workgroups are dispatched round-robin over
  // the 8); with whole 2 x 16 tile groups, 32 consecutive items form one group.
  const int total = gridDim.x;
  const int bid = blockIdx.x;
  const int item = (total & 7) == 0 ? (bid & 7) * (total >> 3) + (bid >> 3) : bid;
  int tm, tn;
  if (a.grouped) {
    const int g = item >> 5, q = item & 31, gpr = a.tiles_n >> 4;
    tm = 2 * (g / gpr) + (q >> 4);
    tn = 16 * (g % gpr) + (q & 15);
  } else {
    tm = item / a.tiles_n;
    tn = item % a.tiles_n;
  }
  const int m0 = tm * kBM, n0 = tn * kBN;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wr = wave & 3, wc = wave >> 2;
  const int cg = lane & 15, kq = lane >> 4;
  const int KB = a.K / kBK;

  // DMA sources.  x: this wave issues stage chunks q = 64*(4*wave + i) + lane; chunk q holds row
  // r = q / 8, k-chunk (q % 8) ^ ((r >> 1) & 7).  Rows past M read row M-1.
  const uint16_t* asrc[kAInstr];
#pragma unroll
  for (int i = 0; i < kAInstr; ++i) {
    const int q = 64 * (kAInstr * wave + i) + lane;
    const int r = q >> 3, c = (q & 7) ^ ((r >> 1) & 7);
    asrc[i] = a.x + (size_t)min(m0 + r, a.M - 1) * a.K + 8 * c;
  }
  // w: this wave issues 8-row block t = wave; lane L loads row 8t + L/8, 16-byte chunk L%8.
  // Chunks past N read column 0 (their outputs are not stored).
  const uint8_t* bsrc[kBInstr];
#pragma unroll
  for (int i = 0; i < kBInstr; ++i) {
    const int t = kBInstr * wave + i;
    const int col = n0 + 16 * (lane & 7);
    bsrc[i] = a.w + (size_t)(8 * t + (lane >> 3)) * a.N + (col + 16 <= a.N ? col : 0);
  }
  auto issue = [&](int kb, uint8_t* st) {
#pragma unroll
    for (int i = 0; i < kAInstr; ++i) dma16(asrc[i] + kb * kBK, st + (kAInstr * wave + i) * 1024);
#pragma unroll
    for (int i = 0; i < kBInstr; ++i)
      dma16(bsrc[i] + (size_t)kb * kBK * a.N, st + kABytes + (kBInstr * wave + i) * kBPitch);
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[rb][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Lane parts of the LDS read addresses (x row 64*wr + i of the first row block, w columns).
  const int i16 = lane & 15;
  const uint32_t a_row = (uint32_t)((64 * wr + i16) * (kBK * 2));
  const uint32_t b_lane = (uint32_t)(kABytes + 64 * wc + 4 * cg);

  for (int s = 0; s < kStages; ++s)
    if (s < KB) issue(s, smem + s * kStage);
  for (int kb = 0; kb < KB; ++kb) {
    uint8_t* st = smem + (kb % kStages) * kStage;
    const int newer = min(kStages - 1, KB - 1 - kb);
    if (newer >= 2)
      wait_vmcnt<2 * kP>();
    else if (newer == 1)
      wait_vmcnt<kP>();
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();  // every wave's DMA for this stage has landed
    const uint32_t sb = lds_addr(st);
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int c = 4 * sub + kq;
      const uint32_t aa = sb + a_row + (uint32_t)((c ^ (i16 >> 1)) * 16);
      const uint32_t ba = sb + b_lane + (uint32_t)((4 * sub + kq) * kBPitch);
      u32x4_v A[4];
      uint32_t Bq[8];
      read_step(aa, ba, A, Bq);
      // B operands: column c of this lane's 4, rows 8*kq + 0..7 as four bf16 pairs.
      u32x4_v B[4];
#pragma unroll
      for (int col = 0; col < 4; ++col) {
        const int sh = 8 * col;
        uint32_t p[4];
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const uint32_t lo = Bq[2 * pp];
          const uint32_t hi = Bq[2 * pp + 1];
          float f0, f1;
          if constexpr (WDT == MX_DTYPE_INT8) {
            f0 = (float)(int8_t)(lo >> sh);
            f1 = (float)(int8_t)(hi >> sh);
          } else {
            f0 = (float)(uint8_t)(lo >> sh);
            f1 = (float)(uint8_t)(hi >> sh);
          }
          p[pp] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
        }
        B[col] = u32x4_v{p[0], p[1], p[2], p[3]};
      }
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int col = 0; col < 4; ++col) acc[rb][col] = mfma(A[rb], B[col], acc[rb][col]);
    }
    __builtin_amdgcn_s_barrier();  // every wave has read this stage
    if (kb + kStages < KB) issue(kb + kStages, st);
  }

  // Epilogue: y = act(acc * s[n] + bias[n]) for this lane's 4 columns.
  const int ncol = n0 + 64 * wc + 4 * cg;
  if (ncol >= a.N) return;
  F4 sc, bi;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    sc.v[c] = load_f(a.scale, ncol + c, a.s_dt);
    bi.v[c] = a.bias ? load_f(a.bias, ncol + c, a.b_dt) : 0.0f;
  }
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + 64 * wr + 16 * rb + 4 * kq + r;
      if (row < a.M) {
        F4 y;
#pragma unroll
        for (int c = 0; c < 4; ++c) y.v[c] = acc[rb][c][r];
        *(uint2*)(a.out + (size_t)row * a.N + ncol) = epilogue4(y, sc, bi, a.act);
      }
    }
  }
}

}  // namespace

bool qdense_gemm_fits(const QDenseDesc& d) {
  auto aligned = [](const void* p, size_t al) { return ((uintptr_t)p % al) == 0; };
  const bool per_channel = d.block_axis == 0 && d.block_size >= d.K;
  return d.M > 16 && d.x_dt == MX_DTYPE_BFLOAT16 && d.scheme == MX_QUANT_LINEAR && !d.zp && per_channel &&
         (d.w_dt == MX_DTYPE_INT8 || d.w_dt == MX_DTYPE_UINT8) && d.K >= kBK && d.K % kBK == 0 && d.N >= 16 &&
         d.N % 16 == 0 && d.M < (1 << 30) && d.K < (1 << 30) && d.N < (1 << 30) && aligned(d.w, 16) &&
         aligned(d.x, 16) && aligned(d.out, 16);
}

int qdense_gemm_run(mx_backend* b, const QDenseDesc& d, const char* name) {
  GemmArgs ga;
  ga.x = (const uint16_t*)d.x;
  ga.w = (const uint8_t*)d.w;
  ga.scale = d.scale;
  ga.bias = d.bias;
  ga.out = (uint16_t*)d.out;
  ga.M = (int)d.M;
  ga.K = (int)d.K;
  ga.N = (int)d.N;
  ga.s_dt = d.s_dt;
  ga.b_dt = d.b_dt;
  ga.act = d.act;
  const int64_t tiles_m = (d.M + kBM - 1) / kBM, tiles_n = (d.N + kBN - 1) / kBN;
  if (tiles_m * tiles_n > (int64_t)1 << 30)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: output too large for the GEMM path");
  ga.tiles_n = (int)tiles_n;
  ga.grouped = (tiles_m % 2 == 0 && tiles_n % 16 == 0) ? 1 : 0;
  const int grid = (int)(tiles_m * tiles_n);
  hipStream_t st = b->stream;
  return launch(b, name, [&] {
    if (d.w_dt == MX_DTYPE_INT8)
      dispatch(qdense_gemm_kernel<MX_DTYPE_INT8>, grid, kThreads, kLds, st, ga);
    else
      dispatch(qdense_gemm_kernel<MX_DTYPE_UINT8>, grid, kThreads, kLds, st, ga);
  });
}

}  // namespace mx
