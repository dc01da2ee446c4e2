// Decode GEMV for the reference's own FusedQuantizedDense formats on gfx950: M <= 4 rows of f32
// (or bf16) activations per launch (up to 64 rows as one launch per group of 4, the weights
// re-read), weights [K, N] in Int8 / Uint8 / Int4 / Uint4, scheme Linear (with or without a zero
// point) or NF4, scales in the reference layout (BlockAxis = 1): scale[k, n/B], shape
// [K, ceil(N/B)], or blocked along K.
//
// Reference semantics: quantizedDenseLinearInt / quantizedDenseNF4
// (internal/gobackend/fusedops/quantizeddense.go:586-650) then the activation epilogue
// (fusedops/dense.go:176-205):
//   y[m,n] = act(bias[n] + sum_k x[m,k] * (w'[k,n] * s[k,n/B] + zp[k,n/B]))
// with w' the integer weight (Linear) or NF4LookupTable[code] (NF4, code = the low 4 bits of the
// stored element).  The scale varies along K, so it cannot be factored out of the K sum: the
// products are f32 FMAs on the VALU, with the per-row factor folded into x first,
//   y = sum_k (x[k] * s[k,b]) * w'[k,n] + sum_k x[k] * zp[k,b].
// Only the summation order and that one rounding differ from the reference loop (results are held
// to the f32 accumulation bound); small problems keep the reference-order kernel.
//
// Layout.  A lane reads one dword of every weight row (4 int8 or 8 int4 columns, CPL), so each
// load instruction of a wave is one contiguous 256-byte row segment and a wave covers 64*CPL
// columns (256 or 512).  A wave takes kGvRows consecutive K rows, all loads issued at entry; a
// workgroup of 8 waves takes 8*kGvRows rows (one K slice) of one column block, so a column block
// has S = ceil(K / (8*kGvRows)) slices.  Each wave stages its own rows of x and its rows of the
// scale (and zero point) blocks that its columns touch into LDS (B >= 32 and B % CPL == 0, so a
// lane's columns share one block and a workgroup touches at most 17 blocks).
//
// Weights are converted with byte converts: int8 as u = w ^ 0x80 (w + 128), int4 as nibbles of
// w ^ 0x8 (w + 8); the offset is removed once at the end with the running sum of x*s.  NF4 codes
// index a 16-entry table in LDS.
//
// Completion.  The waves' tiles are summed through LDS in wave order; with S > 1 every
// workgroup stores its tile and the last one to arrive for the column block adds the S tiles in
// slice order (deterministic), adds the bias, applies the activation (the reference's own) and
// stores f32 or bf16 (the dtype of x).
#include <algorithm>

#include "device_common.h"
#include "mxrt_internal.h"

namespace mx {

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float gv_f32x4;
typedef uint32_t gv_u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGvWaves = 8;
constexpr int kGvWavesWide = 12;  // one-row launches that would otherwise leave CUs with two workgroups
constexpr int kGvPlanCUs = 256;   // CUs the split is planned for (MI355X)
constexpr int kGvThreads = 64 * kGvWaves;
constexpr int kGvRows = 32;                      // K rows per wave
constexpr int kGvSlice = kGvRows * kGvWaves;     // K rows per workgroup
constexpr int kGvMaxRows = 4;                    // M of one launch
constexpr int kGvMaxM = 64;  // larger M runs as launches over groups of kGvMaxRows rows (weights re-read)
constexpr int kGvMinBlock = 32;                  // smallest block size B
constexpr int kGvMaxBlocks = 512 / kGvMinBlock + 1;  // scale blocks one workgroup touches
constexpr int kGvSStride = 32;  // LDS row stride of the staged blocks (a power of two >= kGvMaxBlocks)
constexpr int64_t kGvMinWeights = (int64_t)1 << 20;  // below this the reference-order kernel runs

// Weight kinds: storage dtype x scheme.
enum GvKind { kGvI8 = 0, kGvU8, kGvI4, kGvU4, kGvNF8, kGvNF4 };

struct GemvArgs {
  const void* x;       // [M, K] f32 or bf16
  const uint8_t* w;    // [K, N] storage bytes
  const void* scale;   // [K, nblk]
  const void* zp;      // [K, nblk] or null
  const void* bias;    // [N] or null
  void* out;           // [M, N], dtype of x
  float* partial;      // [S, M, Np] (S > 1)
  uint32_t* counters;  // [column blocks], zero between launches
  int M, K, N, B, S, nblk, act, x_dt, s_dt, zp_dt, b_dt;
  int Np;              // the partial tiles' row stride: N rounded up to 4
};

__device__ __forceinline__ int gv_xcd_swizzle(int bid, int total) {
  // XCD x receives workgroups x, x + 8, ...: total / 8 of them, one more when x < total % 8.
  const int x = bid & 7, base = total >> 3, rem = total & 7;
  return x * base + min(x, rem) + (bid >> 3);
}

// Element idx of a bf16 or f32 array p (null: dummy), read as the aligned 32-bit word holding it
// so that the load is one unconditional instruction whatever the dtype; gv_value picks the element
// once the word has arrived.
struct GvWord {
  uint32_t w, shift;  // shift moves a bf16 element into the high half
};

__device__ __forceinline__ GvWord gv_word(const void* p, int64_t idx, int dt, const void* dummy) {
  const bool bf = dt == MX_DTYPE_BFLOAT16;
  const char* e = p ? (const char*)p + idx * (bf ? 2 : 4) : (const char*)dummy;
  const uint32_t mis = (uint32_t)(uintptr_t)e & 3u;
  return GvWord{*(const uint32_t*)(e - mis), bf ? 16u - 8u * (mis & 2u) : 0u};
}

__device__ __forceinline__ float gv_value(GvWord v, int dt) {
  return dt == MX_DTYPE_BFLOAT16 ? __uint_as_float((v.w << v.shift) & 0xFFFF0000u) : __uint_as_float(v.w);
}

// Byte j of v as a float (v_cvt_f32_ubyte{j}).
template <int J>
__device__ __forceinline__ float gv_ubyte(uint32_t v) {
  return (float)((v >> (8 * J)) & 0xFFu);
}

// Values that must be computed at this point of the program (an empty asm reads and writes them).
template <int MR>
__device__ __forceinline__ void gv_pin(float (&v)[MR]) {
  if constexpr (MR == 1) {
    asm volatile("" : "+v"(v[0]));
  } else {
    asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
  }
}

// AX: the scale layout.  1: the reference's [K, ceil(N/B)] (the scale varies along K and is
// folded into x row by row).  0: blocks of B rows along K, [ceil(K/B), N] (B % 32 == 0 or B >= K,
// so a wave's 32 rows share one group: the wave sums x*w' and x over its rows and applies its
// columns' scale and zero point once).
// UN: rows that start mid-word (N % 8 != 0 for 4-bit weights, N % 4 != 0 for 8-bit ones, K * N
// < 2^31): each lane's word of a row is read as the two aligned words that hold it and a funnel
// shift.
template <int WK, int MR, int AX, int WV = kGvWaves, bool UN = false>
__global__ __launch_bounds__(64 * WV) void qdense_gemv_kernel(GemvArgs a) {
  constexpr int kWv = WV, kThr = 64 * WV, kSlice = kGvRows * WV;
  constexpr bool k4 = WK == kGvI4 || WK == kGvU4 || WK == kGvNF4;
  constexpr bool kNF = WK == kGvNF8 || WK == kGvNF4;
  constexpr int CPL = k4 ? 8 : 4;        // columns per lane
  constexpr int kCols = 64 * CPL;        // columns per workgroup
  constexpr float kOff = WK == kGvI8 ? 128.0f : (WK == kGvI4 ? 8.0f : 0.0f);
  constexpr uint32_t kFlip = WK == kGvI8 ? 0x80808080u : (WK == kGvI4 ? 0x88888888u : 0u);
  // LDS: per wave [x rows][MR] + [rows][blocks] scales (+ zero points) while computing; the
  // waves' tiles [waves][M][kCols] afterwards.
  extern __shared__ __attribute__((aligned(16))) float lds[];
  __shared__ float lut[16];
  __shared__ int s_last;

  const int item = gv_xcd_swizzle(blockIdx.x, gridDim.x);
  const int cb = item / a.S, slice = item % a.S;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int cblk = cb * kCols;
  const int col0 = cblk + lane * CPL;
  const int kw = slice * kSlice + wave * kGvRows;  // first K row of this wave
  const int M = a.M;
  const bool has_zp = a.zp != nullptr;

  // Blocks of the scale rows this workgroup's columns touch: b0 .. b0 + nbw - 1.
  const int b0 = cblk / a.B;
  const int nbw = (min(cblk + kCols, a.N) - 1) / a.B - b0 + 1;
  const int jb = min(col0, a.N - 1) / a.B - b0;  // this lane's block (its columns share it)
  constexpr int kXW = kGvRows * MR;                  // floats of staged x per wave
  constexpr int kSW = AX ? kGvRows * kGvSStride : 0;  // floats of staged scales per wave
  float* xw = lds + wave * (kXW + 2 * kSW);
  float* sw = xw + kXW;
  float* zw = sw + kSW;

  // Staging loads first (x, the scale and zero-point blocks), then every weight row; the
  // staging data is waited for alone (loads complete in order), the weights row by row.
  // Unconditional loads (clamped indices) so that they are all in flight together.
  GvWord xv[MR];
  {
    const int r = lane & (kGvRows - 1);
    const int k = min(kw + r, a.K - 1);
#pragma unroll
    for (int m = 0; m < MR; ++m) xv[m] = gv_word(a.x, (int64_t)min(m, M - 1) * a.K + k, a.x_dt, a.x);
  }
  // AX = 1: the scale/zero-point blocks, staged into LDS.  AX = 0: this lane's columns of its
  // wave's group, kept in registers.
  constexpr int kSL = AX ? (kGvRows * kGvMaxBlocks + 63) / 64 : CPL;  // staging loads per lane
  const int nstage = kGvRows * nbw;
  GvWord sv[kSL], zv[kSL];
  int soff[kSL];  // AX = 1: LDS slot of each staged value (-1: none), computed before the weight loads
#pragma unroll
  for (int i = 0; i < kSL; ++i) {
    int64_t si;
    if constexpr (AX) {
      const int e = min(lane + 64 * i, nstage - 1);
      const int r = e / nbw, j = e - r * nbw;
      const int k = min(kw + r, a.K - 1);
      si = (int64_t)k * a.nblk + b0 + j;
      soff[i] = lane + 64 * i < nstage ? r * kGvSStride + j : -1;
    } else {
      si = (int64_t)(min(kw, a.K - 1) / a.B) * a.N + min(col0 + i, a.N - 1);
      soff[i] = 0;
    }
    sv[i] = gv_word(a.scale, si, a.s_dt, a.x);
    zv[i] = gv_word(a.zp, si, a.zp_dt, a.x);
  }
  const float lut_v = kNF4Table[lane & 15];
  // The staging loads are issued (and so complete) before any weight load; the slots are
  // computed here too (not sunk next to their use, where the arithmetic could wait on a weight).
#pragma unroll
  for (int i = 0; i < kSL; ++i) asm volatile("" : "+v"(soff[i]));
  __builtin_amdgcn_sched_barrier(0);
  const size_t row_bytes = k4 ? (size_t)(a.N >> 1) : (size_t)a.N;
  const size_t lbyte = k4 ? (size_t)(col0 >> 1) : (size_t)col0;
  // Lanes past the row end read its first dword instead (their columns are never stored); rows
  // past K read row K-1 (their x is 0).
  const uint8_t* wp = a.w + (lbyte + 4 <= row_bytes ? lbyte : 0);
  // Issued in row order (the rows are computed in that order and loads complete in order).
  uint32_t wv[kGvRows], wh[UN ? kGvRows : 1];
  // UN: element e = k * N + e0 of the flattened weights (a nibble index for 4-bit weights) is the
  // lane's first; the words are read through a buffer range of the array's size rounded up to 4
  // bytes (the allocation's granule holds those bytes), lanes past N read column 0.
  const uint32_t e0 = col0 < a.N ? (uint32_t)col0 : 0u;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a.w), (short)0,
      UN ? (int)((((uint32_t)a.K * (uint32_t)a.N + (k4 ? 1u : 0u)) / (k4 ? 2u : 1u) + 3u) & ~3u) : 0, 0x00020000);
  auto un_byte = [&](int r) {
    const uint32_t e = (uint32_t)min(kw + r, a.K - 1) * (uint32_t)a.N + e0;
    return k4 ? e >> 1 : e;
  };
  auto un_shift = [&](int r) {
    const uint32_t e = (uint32_t)min(kw + r, a.K - 1) * (uint32_t)a.N + e0;
    return ((k4 ? e >> 1 : e) & 3u) * 8u + (k4 ? (e & 1u) * 4u : 0u);
  };
#pragma unroll
  for (int r = 0; r < kGvRows; ++r) {
    if constexpr (UN) {
      const uint32_t b4 = un_byte(r) & ~3u;
      wv[r] = __builtin_amdgcn_raw_buffer_load_b32(wrs, b4, 0, 0);
      wh[r] = __builtin_amdgcn_raw_buffer_load_b32(wrs, b4 + 4u, 0, 0);
    } else {
      wv[r] = __builtin_nontemporal_load((const uint32_t*)(wp + (size_t)min(kw + r, a.K - 1) * row_bytes));
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  lut[lane & 15] = lut_v;  // every lane: 4 identical writes per entry
  if (lane < kGvRows) {
#pragma unroll
    for (int m = 0; m < MR; ++m) xw[lane * MR + m] = kw + lane < a.K ? gv_value(xv[m], a.x_dt) : 0.0f;
  }
  if constexpr (AX) {
#pragma unroll
    for (int i = 0; i < kSL; ++i) {
      if (soff[i] >= 0) {
        sw[soff[i]] = gv_value(sv[i], a.s_dt);
        zw[soff[i]] = has_zp ? gv_value(zv[i], a.zp_dt) : 0.0f;
      }
    }
  }
  __syncthreads();

  float acc[CPL][MR], sxs[MR], zs[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    sxs[m] = 0.0f;
    zs[m] = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) acc[c][m] = 0.0f;
  }
#pragma unroll
  for (int r = 0; r < kGvRows; ++r) {
    float xr[MR], xs[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) xr[m] = xw[r * MR + m];
    if constexpr (AX) {
      const float s = sw[r * kGvSStride + jb];
#pragma unroll
      for (int m = 0; m < MR; ++m) xs[m] = xr[m] * s;
      // branch-free: the staged zero points are 0 without a zero point
      const float z = zw[r * kGvSStride + jb];
#pragma unroll
      for (int m = 0; m < MR; ++m) zs[m] = __builtin_fmaf(xr[m], z, zs[m]);
    } else {
#pragma unroll
      for (int m = 0; m < MR; ++m) xs[m] = xr[m];
    }
    float wf[CPL];
    const uint32_t v = (UN ? __builtin_amdgcn_alignbit(wh[UN ? r : 0], wv[r], un_shift(r)) : wv[r]) ^ kFlip;
    if constexpr (kNF) {
      if constexpr (k4) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) wf[c] = lut[(v >> (4 * c)) & 15u];
      } else {
#pragma unroll
        for (int c = 0; c < CPL; ++c) wf[c] = lut[(v >> (8 * c)) & 15u];
      }
    } else if constexpr (k4) {
      const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
      wf[0] = gv_ubyte<0>(lo); wf[1] = gv_ubyte<0>(hi);
      wf[2] = gv_ubyte<1>(lo); wf[3] = gv_ubyte<1>(hi);
      wf[4] = gv_ubyte<2>(lo); wf[5] = gv_ubyte<2>(hi);
      wf[6] = gv_ubyte<3>(lo); wf[7] = gv_ubyte<3>(hi);
    } else {
      wf[0] = gv_ubyte<0>(v); wf[1] = gv_ubyte<1>(v);
      wf[2] = gv_ubyte<2>(v); wf[3] = gv_ubyte<3>(v);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (kOff != 0.0f || !AX) sxs[m] += xs[m];
#pragma unroll
      for (int c = 0; c < CPL; ++c) acc[c][m] = __builtin_fmaf(xs[m], wf[c], acc[c][m]);
    }
    // Two rows at a time: the accumulators pass through empty asm statements, so that the
    // products of these rows are computed here (otherwise every row's LDS reads and converted
    // weights are hoisted above the first products and the registers run out).
    if (r & 1) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) gv_pin<MR>(acc[c]);
      gv_pin<MR>(sxs);
      gv_pin<MR>(zs);
      asm volatile("" ::: "memory");
    }
  }
  if constexpr (AX) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float corr = zs[m] - kOff * sxs[m];
#pragma unroll
      for (int c = 0; c < CPL; ++c) acc[c][m] += corr;
    }
  } else {
    // The group's scale and zero point: (sum x*w' - offset * sum x) * s + zp * sum x.
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const float sc = gv_value(sv[c], a.s_dt);
      const float zc = has_zp ? gv_value(zv[c], a.zp_dt) : 0.0f;
#pragma unroll
      for (int m = 0; m < MR; ++m)
        acc[c][m] = __builtin_fmaf(zc, sxs[m], (acc[c][m] - kOff * sxs[m]) * sc);
    }
  }

  // Every wave's tile (rows < M) into LDS as [waves][M][kCols] (over the staging areas, once
  // every wave is done with them); each output then adds the waves in a fixed order.
  __syncthreads();
  float* red = lds;
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (m < M) {
      float* rw = red + ((size_t)wave * M + m) * kCols + lane * CPL;
#pragma unroll
      for (int c = 0; c < CPL; c += 4) *(gv_f32x4*)(rw + c) = gv_f32x4{acc[c][m], acc[c + 1][m], acc[c + 2][m], acc[c + 3][m]};
    }
  }
  __syncthreads();

  constexpr int kQPR = kCols / 4;  // quads per tile row
  const int MC = M * kCols, NQ = M * kQPR;
  const int t = threadIdx.x;
  auto finish_quad = [=](int m, int col, gv_f32x4 y) {
    if (col >= a.N) return;
    const int64_t o = (int64_t)m * a.N + col;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (col + e >= a.N) break;
      const float b = a.bias ? load_f(a.bias, col + e, a.b_dt) : 0.0f;
      store_f(a.out, o + e, a.x_dt, act_ref(y[e] + b, a.act));
    }
  };
  auto wave_sum = [=](int g) {
    gv_f32x4 y = *(const gv_f32x4*)(red + 4 * g);
#pragma unroll
    for (int w = 1; w < kWv; ++w) y += *(const gv_f32x4*)(red + w * MC + 4 * g);
    return y;
  };

  if (a.S == 1) {
    for (int g = t; g < NQ; g += kThr) finish_quad(g / kQPR, cblk + 4 * (g % kQPR), wave_sum(g));
    return;
  }

  // Split K: store this slice's tile as [slice][M][N] (16-byte stores with the agent-scope
  // coherence bit sc1), wait until the stores have completed, then count the arrival; only the
  // last arriver reads the tiles back, with loads that carry the same bit.  The tiles' rows are
  // Np = N rounded up to 4 floats apart, so a quad is whole or past the end.
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      a.partial, (short)0, (int)((size_t)a.S * M * a.Np * sizeof(float)), 0x00020000);
  constexpr int kSc1 = 16;  // cache-policy operand of the buffer intrinsics: sc1
  for (int g = t; g < NQ; g += kThr) {
    const int m = g / kQPR, col = cblk + 4 * (g % kQPR);
    if (col < a.N)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(gv_u32x4, wave_sum(g)), prs,
                                            (unsigned)(((slice * M + m) * a.Np + col) * 4), 0, kSc1);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&a.counters[cb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == (uint32_t)a.S - 1u;
    if (last) __hip_atomic_store(&a.counters[cb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  constexpr int kSl = 16;
  for (int g = t; g < NQ; g += kThr) {
    const int m = g / kQPR, col = cblk + 4 * (g % kQPR);
    const int c = min(col, a.Np - 4);
    gv_f32x4 y = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < a.S; s0 += kSl) {
      gv_f32x4 v[kSl];
#pragma unroll
      for (int u = 0; u < kSl; ++u) {
        const int s = min(s0 + u, a.S - 1);
        v[u] = __builtin_bit_cast(gv_f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                prs, (unsigned)(((s * M + m) * a.Np + c) * 4), 0, kSc1));
      }
#pragma unroll
      for (int u = 0; u < kSl; ++u)
        if (s0 + u < a.S) y += v[u];
    }
    finish_quad(m, col, y);
  }
}

// ---------------------------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------------------------
static int gemv_kind(const QDenseDesc& d) {
  const bool nf4 = d.scheme == MX_QUANT_NF4;
  switch (d.w_dt) {
    case MX_DTYPE_INT8: return nf4 ? kGvNF8 : kGvI8;
    case MX_DTYPE_UINT8: return nf4 ? kGvNF8 : kGvU8;
    case MX_DTYPE_INT4: return nf4 ? kGvNF4 : kGvI4;
    case MX_DTYPE_UINT4: return nf4 ? kGvNF4 : kGvU4;
    default: return -1;
  }
}

static bool gv_float_dt(int dt) { return dt == MX_DTYPE_FLOAT32 || dt == MX_DTYPE_BFLOAT16; }

bool qdense_gemv_fits(const QDenseDesc& d) {
  if (d.M < 1 || d.M > kGvMaxM) return false;
  if (d.scheme != MX_QUANT_LINEAR && d.scheme != MX_QUANT_NF4) return false;
  const int kind = gemv_kind(d);
  if (kind < 0 || !gv_float_dt(d.x_dt) || !gv_float_dt(d.s_dt)) return false;
  if (d.zp && !gv_float_dt(d.zp_dt)) return false;
  if (d.bias && !gv_float_dt(d.b_dt)) return false;
  const bool packed = dtype_is_packed(d.w_dt);
  const int cpl = packed ? 8 : 4;
  auto aligned = [](const void* p, size_t al) { return ((uintptr_t)p % al) == 0; };
  const bool blocks = d.block_axis == 1 ? d.block_size >= kGvMinBlock && d.block_size % cpl == 0
                                        : d.block_size % kGvRows == 0 || d.block_size >= d.K;
  // Rows that start mid-word (other N) take the kernel's two-word loads, within 2^31 elements.
  return d.K >= 1 && d.K * d.N >= kGvMinWeights && d.K < (int64_t)1 << 30 && d.N < (int64_t)1 << 30 &&
         (d.N % (packed ? 8 : 4) == 0 || d.K * d.N < ((int64_t)1 << 31)) && blocks && aligned(d.w, 4) &&
         aligned(d.out, d.x_dt == MX_DTYPE_FLOAT32 ? 16 : 8);
}

template <int WK, int AX>
static void gemv_launch_ax(const GemvArgs& ga, int waves, int grid, size_t lds, hipStream_t st) {
  if (ga.N % (WK == kGvI4 || WK == kGvU4 || WK == kGvNF4 ? 8 : 4) != 0) {  // rows start mid-word
    if (ga.M == 1)
      dispatch(qdense_gemv_kernel<WK, 1, AX, kGvWaves, true>, grid, kGvThreads, lds, st, ga);
    else
      dispatch(qdense_gemv_kernel<WK, kGvMaxRows, AX, kGvWaves, true>, grid, kGvThreads, lds, st, ga);
    return;
  }
  if (ga.M == 1 && waves == kGvWavesWide)
    dispatch(qdense_gemv_kernel<WK, 1, AX, kGvWavesWide>, grid, 64 * kGvWavesWide, lds, st, ga);
  else if (ga.M == 1)
    dispatch(qdense_gemv_kernel<WK, 1, AX>, grid, kGvThreads, lds, st, ga);
  else
    dispatch(qdense_gemv_kernel<WK, kGvMaxRows, AX>, grid, kGvThreads, lds, st, ga);
}

template <int WK>
static void gemv_launch(const GemvArgs& ga, int axis, int waves, int grid, size_t lds, hipStream_t st) {
  if (axis == 1)
    gemv_launch_ax<WK, 1>(ga, waves, grid, lds, st);
  else
    gemv_launch_ax<WK, 0>(ga, waves, grid, lds, st);
}

static int gemv_run_rows(mx_backend* b, const QDenseDesc& d, const char* name);

int qdense_gemv_run(mx_backend* b, const QDenseDesc& d, const char* name) {
  // Groups of kGvMaxRows rows of x and of the output, one launch each (the split-K counters are
  // back at zero after every launch, and the launches are ordered on the stream).
  const size_t xe = d.x_dt == MX_DTYPE_FLOAT32 ? 4 : 2;
  for (int64_t m0 = 0; m0 < d.M; m0 += kGvMaxRows) {
    QDenseDesc g = d;
    g.M = std::min<int64_t>(kGvMaxRows, d.M - m0);
    g.x = (const char*)d.x + (size_t)m0 * d.K * xe;
    g.out = (char*)d.out + (size_t)m0 * d.N * xe;
    MX_TRY(gemv_run_rows(b, g, name));
  }
  return MX_OK;
}

static int gemv_run_rows(mx_backend* b, const QDenseDesc& d, const char* name) {
  const bool packed = dtype_is_packed(d.w_dt);
  const int64_t cols = packed ? 512 : 256;
  const int64_t nb = (d.N + cols - 1) / cols;
  // One row: twelve-wave workgroups where the 8-wave grid would give some CUs two workgroups and
  // twelve waves give one workgroup per CU on at least three quarters of them (planned for
  // MI355X's 256 CUs whatever the device reports, so the split, and the bits, depend on the
  // shape only).
  const int64_t S8 = (d.K + kGvSlice - 1) / kGvSlice;
  const int64_t SW = (d.K + kGvRows * kGvWavesWide - 1) / (kGvRows * kGvWavesWide);
  const bool unaligned = d.N % (packed ? 8 : 4) != 0;  // eight-wave kernels only
  const int waves = !unaligned && d.M == 1 && nb * S8 > kGvPlanCUs && nb * SW <= kGvPlanCUs &&
                            4 * nb * SW >= 3 * kGvPlanCUs
                        ? kGvWavesWide
                        : kGvWaves;
  const int64_t Np = (d.N + 3) / 4 * 4;
  const int64_t S = waves == kGvWaves ? S8 : SW;
  const size_t counter_bytes = 64 * 1024;
  if ((size_t)nb * 4 > counter_bytes || nb * S > (int64_t)1 << 30 || S * d.M * Np * 4 >= (int64_t)1 << 31)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: N=%lld too large for the GEMV path", (long long)d.N);
  GemvArgs ga;
  ga.x = d.x;
  ga.w = (const uint8_t*)d.w;
  ga.scale = d.scale;
  ga.zp = d.zp;
  ga.bias = d.bias;
  ga.out = d.out;
  ga.partial = nullptr;
  ga.counters = nullptr;
  if (S > 1) {
    void* scratch = nullptr;
    MX_TRY(ensure_scratch(b, counter_bytes + (size_t)S * d.M * Np * sizeof(float), &scratch));
    ga.counters = (uint32_t*)scratch;
    ga.partial = (float*)((char*)scratch + counter_bytes);
  }
  ga.M = (int)d.M;
  ga.K = (int)d.K;
  ga.N = (int)d.N;
  ga.Np = (int)Np;
  ga.B = (int)std::min<int64_t>(d.block_size, d.block_axis == 1 ? d.N : d.K);
  ga.S = (int)S;
  ga.nblk = (int)((d.N + d.block_size - 1) / d.block_size);
  ga.act = d.act;
  ga.x_dt = d.x_dt;
  ga.s_dt = d.s_dt;
  ga.zp_dt = d.zp_dt;
  ga.b_dt = d.b_dt;
  const int mr = d.M == 1 ? 1 : kGvMaxRows;
  const size_t stage =
      (size_t)waves * (kGvRows * mr + (d.block_axis == 1 ? 2 * kGvRows * kGvSStride : 0)) * sizeof(float);
  const size_t tiles = (size_t)waves * d.M * cols * sizeof(float);
  const size_t lds = std::max(stage, tiles);
  const int grid = (int)(nb * S);
  hipStream_t st = b->stream;
  return launch(b, name, [&] {
    switch (gemv_kind(d)) {
      case kGvI8: gemv_launch<kGvI8>(ga, d.block_axis, waves, grid, lds, st); break;
      case kGvU8: gemv_launch<kGvU8>(ga, d.block_axis, waves, grid, lds, st); break;
      case kGvI4: gemv_launch<kGvI4>(ga, d.block_axis, waves, grid, lds, st); break;
      case kGvU4: gemv_launch<kGvU4>(ga, d.block_axis, waves, grid, lds, st); break;
      case kGvNF8: gemv_launch<kGvNF8>(ga, d.block_axis, waves, grid, lds, st); break;
      default: gemv_launch<kGvNF4>(ga, d.block_axis, waves, grid, lds, st); break;
    }
  });
}

}  // namespace mx
