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
// in blocks of 64 (two 32-row steps of v_mfma_f32_16x16x32_bf16).
//   - x: a 3-stage LDS ring of [256 rows][64 k] bf16 tiles filled by direct global->LDS loads
//     (16 bytes per lane) issued two blocks ahead; 16-byte chunks are XOR-swizzled within each
//     row by (row >> 1) & 7 so that an MFMA operand read (16 rows) hits distinct banks.
//   - w: each thread loads 4 rows x 4 columns of int8 per block into registers (two blocks
//     ahead; a wave's load covers 2 rows x 128 contiguous bytes), converts them exactly to bf16
//     (|w| < 256 has at most 8 significant bits) and writes them transposed into a bf16 tile
//     Bt[128 columns][64 k], double-buffered, whose 16-byte k-chunks are XOR-swizzled by
//     (column >> 2) & 7 (conflict-free B-operand reads: 8 consecutive k of one column).
//     Block kb + 1 is dequantised between the two MFMA steps of block kb, so the weights are
//     converted once per workgroup and the conversion overlaps the matrix cores.
// One barrier per K block publishes the next Bt buffer and retires the reads of the current ring
// stage, which is then refilled.  Every load is issued unconditionally (block indices past the
// end are clamped), so the number of loads in flight is the same in every iteration and the
// explicit vmcnt waits are exact.  Lane (cg = lane % 16, kq = lane / 16) ends with rows 4*kq + r
// of each 16-row block and the 4 consecutive columns 4*cg .. 4*cg + 3 of its wave's 64; the
// epilogue applies scale, bias and activation and writes 8-byte bf16 runs.
// Tile order: every XCD (workgroups are dispatched round-robin over the 8) takes a 2 x 16 block
// of tiles, so its L2 serves the x rows and w columns they share.
//
// The LDS accesses are inline assembly: LDS reads or writes written in C++ after the direct
// global->LDS loads would make the compiler wait for every outstanding load (vmcnt(0)) first,
// emptying the prefetch ring.  The asm blocks wait for their own results (lgkmcnt).
#include <algorithm>
#include <type_traits>

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
constexpr int kABytes = kBM * kBK * 2;              // 32 KB per ring stage
constexpr int kBtBytes = kBN * kBK * 2;             // 16 KB per Bt buffer
constexpr int kLds = kStages * kABytes + 2 * kBtBytes;
constexpr int kAInstr = kABytes / (kWaves * 1024);  // direct loads per wave per stage
constexpr int kWLoads = 4;                          // w loads per thread per block
static_assert(kAInstr * kWaves * 1024 == kABytes, "x load split");
static_assert(kBK * kBN == 16 * kThreads, "conversion: 16 weights per thread");

struct GemmArgs {
  const uint16_t* x;  // [M, K] bf16
  const uint8_t* w;   // [K, N] int8 / uint8
  const void* scale;  // [N]
  const void* bias;   // [N] or null
  uint16_t* out;      // [M, N] bf16
  int M, K, N, s_dt, b_dt, act, tiles_n, grouped;
};

__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
  __builtin_amdgcn_global_load_lds((gbl_void_ptr)const_cast<void*>(src), (lds_void_ptr)(uintptr_t)lds, 16, 0, 0);
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

// Four bf16 k-values of each of four consecutive columns of Bt (rows 128 bytes apart).
__device__ __forceinline__ void write_bt4(uint32_t addr, const u32x2_v (&v)[4]) {
  asm volatile(
      "ds_write_b64 %0, %1 offset:0\n\t"
      "ds_write_b64 %0, %2 offset:128\n\t"
      "ds_write_b64 %0, %3 offset:256\n\t"
      "ds_write_b64 %0, %4 offset:384\n\t"
      "s_waitcnt lgkmcnt(0)"
      :
      : "v"(addr), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3])
      : "memory");
}

// One K step's operands: the wave's 4 x-row blocks (16 bytes each, 2 KB apart) and its 4
// Bt-column blocks (16 bytes each, 128 bytes apart).
__device__ __forceinline__ void read_step(uint32_t aa, uint32_t ba, u32x4_v (&A)[4], u32x4_v (&B)[4]) {
  asm volatile(
      "ds_read_b128 %0, %8 offset:0\n\t"
      "ds_read_b128 %1, %8 offset:2048\n\t"
      "ds_read_b128 %2, %8 offset:4096\n\t"
      "ds_read_b128 %3, %8 offset:6144\n\t"
      "ds_read_b128 %4, %9 offset:0\n\t"
      "ds_read_b128 %5, %9 offset:128\n\t"
      "ds_read_b128 %6, %9 offset:256\n\t"
      "ds_read_b128 %7, %9 offset:384\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(A[0]), "=&v"(A[1]), "=&v"(A[2]), "=&v"(A[3]), "=&v"(B[0]), "=&v"(B[1]), "=&v"(B[2]), "=&v"(B[3])
      : "v"(aa), "v"(ba)
      : "memory");
}

// Workgroup barrier.  The LDS accesses around it are asm blocks that have waited for their own
// completion, so the barrier alone orders them.
__device__ __forceinline__ void barrier() { __builtin_amdgcn_s_barrier(); }

// act(v * s + b) rounded to bf16, for a compile-time activation.
template <int ACT>
__device__ __forceinline__ uint32_t scaled_act_bf16(float v, float s, float b) {
  return f32_to_bf16(act_fast(v * s + b, ACT));
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
          o[c / 2] = scaled_act_bf16<ACT>(acc[rb][c][r], sc[c], bi[c]) |
                     (scaled_act_bf16<ACT>(acc[rb][c + 1][r], sc[c + 1], bi[c + 1]) << 16);
        *(uint2*)(out + (size_t)row * N + ncol) = make_uint2(o[0], o[1]);
      }
    }
  }
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
  const size_t N = (size_t)a.N;

  // x direct loads: this wave fills stage chunks q = 64*(4*wave + i) + lane; chunk q holds row
  // r = q / 8, k-chunk (q % 8) ^ ((r >> 1) & 7).  Rows past M read row M-1.
  const uint16_t* asrc[kAInstr];
#pragma unroll
  for (int i = 0; i < kAInstr; ++i) {
    const int q = 64 * (kAInstr * wave + i) + lane;
    const int r = q >> 3, c = (q & 7) ^ ((r >> 1) & 7);
    asrc[i] = a.x + (size_t)min(m0 + r, a.M - 1) * a.K + 8 * c;
  }
  const uint32_t smem_base = lds_addr(smem);
  const uint32_t bt_base = smem_base + kStages * kABytes;
  auto issue_x = [&](int kb) {
    const uint32_t st = smem_base + (uint32_t)((kb % kStages) * kABytes);
    kb = min(kb, KB - 1);
#pragma unroll
    for (int i = 0; i < kAInstr; ++i) dma16(asrc[i] + kb * kBK, st + (uint32_t)((kAInstr * wave + i) * 1024));
  };
  // w: thread t converts columns 4*cq .. 4*cq + 3 and rows 4*j .. 4*j + 3 of each block; the 32
  // threads of a j read 128 contiguous bytes of a row.  Columns past N read column 0 (their
  // outputs are not stored).
  const int t = threadIdx.x, cq = t & 31, j = t >> 5;
  const int wcol = n0 + 4 * cq + 4 <= a.N ? n0 + 4 * cq : 0;
  const uint8_t* wsrc = a.w + (size_t)(4 * j) * N + wcol;
  const uint32_t cv_addr = bt_base + (uint32_t)(4 * cq * (kBK * 2) + (((j >> 1) ^ (cq & 7)) << 4) + ((j & 1) << 3));
  auto load_w = [&](int kb, uint32_t (&dst)[kWLoads]) {
    kb = min(kb, KB - 1);
#pragma unroll
    for (int e = 0; e < kWLoads; ++e)
      dst[e] = __builtin_nontemporal_load((const uint32_t*)(wsrc + (size_t)(kb * kBK + e) * N));
  };
  auto convert = [&](const uint32_t (&w4)[kWLoads], int buf) {
    u32x2_v v[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float f[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (WDT == MX_DTYPE_INT8)
          f[e] = (float)(int8_t)(w4[e] >> (8 * c));
        else
          f[e] = (float)(uint8_t)(w4[e] >> (8 * c));
      }
      v[c] = u32x2_v{__builtin_amdgcn_perm(__float_as_uint(f[1]), __float_as_uint(f[0]), 0x07060302u),
                     __builtin_amdgcn_perm(__float_as_uint(f[3]), __float_as_uint(f[2]), 0x07060302u)};
    }
    write_bt4(cv_addr + (uint32_t)(buf * kBtBytes), v);
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[rb][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // MFMA operand reads: x row 64*wr + cg of the first row block; Bt column 64*wc + 4*cg.
  const uint32_t a_row = (uint32_t)((64 * wr + cg) * (kBK * 2));
  const uint32_t b_col = bt_base + (uint32_t)((64 * wc + 4 * cg) * (kBK * 2));
  auto mma_step = [&](int kb, int buf, int sub) {
    const uint32_t sb = smem_base + (uint32_t)((kb % kStages) * kABytes);
    const int kc = 4 * sub + kq;  // 16-byte k-chunk of this lane
    const uint32_t aa = sb + a_row + (uint32_t)((kc ^ (cg >> 1)) << 4);
    const uint32_t ba = b_col + (uint32_t)(buf * kBtBytes) + (uint32_t)((kc ^ (cg & 7)) << 4);
    u32x4_v A[4], B[4];
    read_step(aa, ba, A, B);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[rb][c] = mfma(A[rb], B[c], acc[rb][c]);
  };

  // Loads in flight, in issue order, at the end of block kb (before its wait): x block kb + 1,
  // w block kb + 2, x block kb + 2, w block kb + 3.  Block kb + 1's x is complete once only the
  // three newer groups are outstanding.
  constexpr int kWaitX = kWLoads + kAInstr + kWLoads;
  uint32_t wv[2][kWLoads];  // [ring slot][row]: w of blocks kb + 1 and kb + 2
  // One K block; S = kb % 2 (compile-time, so the w ring is indexed statically).  On entry Bt
  // buffer S holds block kb, wv[S ^ 1] holds block kb + 1's int8 weights and x block kb is in its
  // ring stage.
  auto block = [&](int kb, auto slot) {
    constexpr int S = decltype(slot)::value;
    mma_step(kb, S, 0);
    __builtin_amdgcn_sched_barrier(0);
    convert(wv[S ^ 1], S ^ 1);
    load_w(kb + 3, wv[S ^ 1]);
    __builtin_amdgcn_sched_barrier(0);
    mma_step(kb, S, 1);
    wait_vmcnt<kWaitX>();
    barrier();  // Bt buffer S ^ 1 published; every read of x stage kb and Bt buffer S retired
    issue_x(kb + 3);
  };

  issue_x(0);
  load_w(0, wv[0]);
  issue_x(1);
  load_w(1, wv[1]);
  issue_x(2);
  convert(wv[0], 0);  // waits (compiler) for block 0's w
  load_w(2, wv[0]);
  // In flight now: x0, x1, w1, x2, w2 (w0 done); x0 complete once x1, w1, x2, w2 may remain.
  wait_vmcnt<kAInstr + kWLoads + kAInstr + kWLoads>();
  barrier();
  int kb = 0;
  for (; kb + 1 < KB; kb += 2) {
    block(kb, std::integral_constant<int, 0>{});
    block(kb + 1, std::integral_constant<int, 1>{});
  }
  if (kb < KB) block(kb, std::integral_constant<int, 0>{});
  wait_vmcnt<0>();  // drain the clamped prefetches before the workgroup's LDS is released

  // Epilogue: y = act(acc * s[n] + bias[n]) for this lane's 4 columns.
  const int ncol = n0 + 64 * wc + 4 * cg;
  if (ncol >= a.N) return;
  float sc[4], bi[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    sc[c] = load_f(a.scale, ncol + c, a.s_dt);
    bi[c] = a.bias ? load_f(a.bias, ncol + c, a.b_dt) : 0.0f;
  }
  const int row0 = m0 + 64 * wr + 4 * kq;
  switch (a.act) {
    case MX_ACT_GELU: store_tile<MX_ACT_GELU>(acc, sc, bi, a.out, row0, a.M, N, ncol); break;
    case MX_ACT_RELU: store_tile<MX_ACT_RELU>(acc, sc, bi, a.out, row0, a.M, N, ncol); break;
    case MX_ACT_SILU: store_tile<MX_ACT_SILU>(acc, sc, bi, a.out, row0, a.M, N, ncol); break;
    case MX_ACT_HARDSWISH: store_tile<MX_ACT_HARDSWISH>(acc, sc, bi, a.out, row0, a.M, N, ncol); break;
    case MX_ACT_TANH: store_tile<MX_ACT_TANH>(acc, sc, bi, a.out, row0, a.M, N, ncol); break;
    default: store_tile<MX_ACT_NONE>(acc, sc, bi, a.out, row0, a.M, N, ncol); break;
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
