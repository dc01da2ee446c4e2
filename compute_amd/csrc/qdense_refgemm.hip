// FusedQuantizedDense at prefill size for the layouts the bf16 matrix-core GEMM does not take: the
// reference's own scale layout [K, ceil(N/B)] (BlockAxis = 1), f32 x, zero points and NF4
// (fused_ops.go:204-234; quantizeddense.go:586-650).  The dequantisation is fused into the
// contraction: each K block of the weights is dequantised in registers and written to LDS as f32,
// and the products run on the f32 matrix cores (v_mfma_f32_16x16x4_f32).  No f32 copy of the
// weight matrix is ever made.
//
// Per term the weight factor is formed as the reference forms it and rounded once to f32: w*s,
// w*s + zp (two roundings) or nf4[w]*s; the product with x is x*(w*s) where the reference rounds
// (x*w)*s, and the sums run in the matrix cores' order, so the result stays within the f32
// accumulation bound of the reference's sum.  The bias is added after the sum (the reference
// starts its sum from the bias), then the reference activation (act_ref) and the output dtype.
//
// Tiling: a workgroup of 4 waves owns a 128 x 128 output tile (2 x 2 waves of 64 x 64, each 4 x 4
// MFMA tiles of 16 x 16), K in blocks of 32.  Block kb + 1 is requested into registers before
// block kb is multiplied, then dequantised into the other of two LDS buffers:
//   A  x rows [m0, m0 + 128) x 32 k, f32, rows padded to 144 bytes;
//   B  the weights' 32 rows x 128 columns, dequantised to f32, rows padded to 520 bytes.
// MFMA step t (0..7) of a block contracts k = 8 g + t, g = lane / 16: a lane reads 8 consecutive
// k of its A row (two 16-byte reads) and k = 8 g + t of its B column (4-byte reads, the 520-byte
// rows put the four lane groups on disjoint banks).  A thread dequantises 16 consecutive columns
// of one weight row per block (16 int8 bytes or 8 Int4 bytes, one 16-byte load).
//
// Tiles are ordered so that each XCD takes a contiguous run of tiles, M-major: the x rows of its
// tiles stay in that XCD's L2 while all of its N tiles are computed.
#include "device_common.h"
#include "mxrt_internal.h"

namespace mx {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_v __attribute__((ext_vector_type(2)));

constexpr int kRgBM = 128, kRgBN = 128, kRgBK = 32, kRgThreads = 256;
constexpr int kRgAS = kRgBK * 4 + 16;          // LDS bytes per A row
constexpr int kRgBS = kRgBN * 4 + 8;           // LDS bytes per B row
constexpr int kRgABytes = kRgBM * kRgAS;
constexpr int kRgBuf = kRgABytes + kRgBK * kRgBS;  // one LDS buffer (A then B)

// How a thread finds the scales (and zero points) of its 16 columns in one weight row k.
enum RgScaleMode {
  kRgCols = 0,  // one scale per column of a scale row: [ceil(K/B), N] (BlockAxis 0) or [N]
  kRgBlk = 1,   // [K, ceil(N/B)] with B >= 16: at most two blocks per 16 columns
  kRgAny = 2    // [K, ceil(N/B)] with B < 16: a block per column
};

struct RefGemmArgs {
  const void* x;      // [M, K] f32 or bf16
  const uint8_t* w;   // [K, N] storage bytes
  const void* scale;  // see RgScaleMode
  const void* zp;     // same layout as scale, or null
  const void* bias;   // [N] or null
  void* out;          // [M, N], x's dtype
  int M, K, N;
  int x_dt, s_dt, zp_dt, b_dt, act, nf4;
  int B;            // block size along the scale's blocked axis
  int nb;           // scale row length for kRgBlk / kRgAny: ceil(N / B)
  int tiles_n, tiles, per_xcd;
};

// Element i of an f32 or bf16 array as f32.
__device__ __forceinline__ float rg_load(const void* p, int64_t i, int dt) {
  return dt == MX_DTYPE_BFLOAT16 ? bf16_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

// PLAIN: f32 x, linear scheme, no zero points: the common case, with every dtype test of the
// general kernel resolved at compile time.
template <int WDT, int SM, bool PLAIN>
__global__ __launch_bounds__(kRgThreads, 2) void qdense_refgemm_kernel(RefGemmArgs a) {
  constexpr bool kI4 = WDT == MX_DTYPE_INT4 || WDT == MX_DTYPE_UINT4;
  constexpr bool kSigned = WDT == MX_DTYPE_INT4 || WDT == MX_DTYPE_INT8;
  if constexpr (PLAIN) {
    a.x_dt = MX_DTYPE_FLOAT32;
    a.zp = nullptr;
    a.nf4 = 0;
  }
  __shared__ __attribute__((aligned(16))) char sm[2][kRgBuf];
  __shared__ float nf4[16];

  // XCD-contiguous tile order: workgroups are dispatched round-robin over the 8 XCDs.
  const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int tile = xcd * a.per_xcd + j;
  if (j >= a.per_xcd || tile >= a.tiles) return;
  const int m0 = (tile / a.tiles_n) * kRgBM, n0 = (tile % a.tiles_n) * kRgBN;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1, r = lane & 15, g = lane >> 4;
  const int M = a.M, K = a.K, N = a.N;
  if (t < 16) nf4[t] = kNF4Table[t];

  // ---- This thread's share of the loads of a K block.
  // x: f32 chunks c = t + 256 p (p < 4): row c / 8, k 4 (c % 8) .. +4; bf16 chunks (p < 2): row
  // c / 4, k 8 (c % 4) .. +8.  Rows past M read row M - 1 and store zeros.
  const bool xbf = a.x_dt == MX_DTYPE_BFLOAT16;
  // Weights: row k = 32 kb + t / 8 of the block, columns nc .. nc + 15 with nc = n0 + 16 (t % 8).
  const int wrow = t >> 3, nc = n0 + 16 * (t & 7);
  const bool ncol_ok = nc < N;  // N % 16 == 0: the 16 columns are all in range or all past it
  const int ncl = ncol_ok ? nc : 0;
  // Scale blocks of the 16 columns (kRgBlk: blo for columns < jsplit, blo + 1 after).
  const int blo = SM == kRgCols ? 0 : ncl / a.B;
  const int jsplit = SM == kRgBlk ? min(16, (blo + 1) * a.B - ncl) : 16;

  // Every load below is unconditional (dtype choices only select addresses or bits), so that the
  // compiler waits for a block's loads where they are used, not where they are issued.
  const bool sbf = a.s_dt == MX_DTYPE_BFLOAT16, zbf = a.zp_dt == MX_DTYPE_BFLOAT16;
  struct Regs {
    u32x4_v x[4];
    u32x4_v w;       // 16 bytes (int8) or 8 (Int4, in .xy)
    uint32_t s[16];  // raw scale words (kRgCols: 16 f32 or 8 bf16 pairs; kRgBlk: 2; kRgAny: 16)
    uint32_t z[16];  // the same for zero points
    uint32_t ssh[16], zsh[16];  // kRgBlk / kRgAny: shift moving a bf16 element to the high half
  };
  // The aligned word holding element i of an f32 or bf16 array, and its shift.
  auto word = [&](const void* p, int64_t i, bool bf, uint32_t& w, uint32_t& sh) __attribute__((always_inline)) {
    const uintptr_t ad = (uintptr_t)p + (uintptr_t)i * (bf ? 2 : 4);
    w = *(const uint32_t*)(ad & ~(uintptr_t)3);
    sh = bf && (ad & 2) == 0 ? 16u : 0u;
  };
  auto gload = [&](int kb, Regs& R) __attribute__((always_inline)) {
    const int k0 = kb * kRgBK;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // bf16 x needs two chunks per thread; the other two reload them (in bounds, unused).
      const int c = t + 256 * (xbf ? (p & 1) : p);
      const int row = xbf ? c >> 2 : c >> 3, kc = xbf ? (c & 3) * 8 : (c & 7) * 4;
      const int m = min(m0 + row, M - 1);
      const int k = min(k0 + kc, K - (xbf ? 8 : 4));
      R.x[p] = *(const u32x4_v*)((const char*)a.x + ((int64_t)m * K + k) * (xbf ? 2 : 4));
    }
    const int k = min(k0 + wrow, K - 1);
    const char* wp = (const char*)a.w + ((int64_t)k * N + ncl) / (kI4 ? 2 : 1);
    if constexpr (kI4) {
      const u32x2_v v = *(const u32x2_v*)wp;
      R.w = u32x4_v{v[0], v[1], 0u, 0u};
    } else {
      R.w = *(const u32x4_v*)wp;
    }
    if constexpr (SM == kRgCols) {
      // 16 consecutive scales: four 16-byte loads of f32, two of bf16 (the other two repeat them).
      const int64_t si = (int64_t)(k / a.B) * N + ncl;
      const char* sp = (const char*)a.scale + si * (sbf ? 2 : 4);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4_v v = *(const u32x4_v*)(sp + 16 * (sbf ? (q & 1) : q));
#pragma unroll
        for (int e = 0; e < 4; ++e) R.s[4 * q + e] = v[e];
      }
      if (a.zp) {
        const char* zq = (const char*)a.zp + si * (zbf ? 2 : 4);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4_v v = *(const u32x4_v*)(zq + 16 * (zbf ? (q & 1) : q));
#pragma unroll
          for (int e = 0; e < 4; ++e) R.z[4 * q + e] = v[e];
        }
      }
    } else if constexpr (SM == kRgBlk) {
      const int64_t si = (int64_t)k * a.nb + blo;
      const int64_t s2 = min<int64_t>(si + 1, (int64_t)k * a.nb + a.nb - 1);
      word(a.scale, si, sbf, R.s[0], R.ssh[0]);
      word(a.scale, s2, sbf, R.s[1], R.ssh[1]);
      if (a.zp) {
        word(a.zp, si, zbf, R.z[0], R.zsh[0]);
        word(a.zp, s2, zbf, R.z[1], R.zsh[1]);
      }
    } else {
      int b = blo, rem = ncl - blo * a.B;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t si = (int64_t)k * a.nb + b;
        word(a.scale, si, sbf, R.s[e], R.ssh[e]);
        if (a.zp) word(a.zp, si, zbf, R.z[e], R.zsh[e]);
        if (++rem == a.B) {
          rem = 0;
          ++b;
        }
      }
    }
  };

  // Dequantise the registers of block kb into LDS buffer `buf` (zeros for rows past M, k past
  // K and columns past N).
  auto lstore = [&](int kb, const Regs& R, int buf) __attribute__((always_inline)) {
    const int k0 = kb * kRgBK;
    char* As = sm[buf];
    char* Bs = sm[buf] + kRgABytes;
    const u32x4_v zero4 = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if (!xbf) {
        const int c = t + 256 * p, row = c >> 3, kc = (c & 7) * 4;
        const bool ok = m0 + row < M && k0 + kc < K;
        *(u32x4_v*)(As + row * kRgAS + kc * 4) = ok ? R.x[p] : zero4;
      } else if (p < 2) {
        const int c = t + 256 * p, row = c >> 2, kc = (c & 3) * 8;
        const bool ok = m0 + row < M && k0 + kc < K;
        u32x4_v lo, hi;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          lo[2 * e] = R.x[p][e] << 16;
          lo[2 * e + 1] = R.x[p][e] & 0xFFFF0000u;
          hi[2 * e] = R.x[p][2 + e] << 16;
          hi[2 * e + 1] = R.x[p][2 + e] & 0xFFFF0000u;
        }
        *(u32x4_v*)(As + row * kRgAS + kc * 4) = ok ? lo : zero4;
        *(u32x4_v*)(As + row * kRgAS + kc * 4 + 16) = ok ? hi : zero4;
      }
    }
    const bool ok = ncol_ok && k0 + wrow < K;
    const uint32_t smask = sbf ? 0xFFFF0000u : ~0u, zmask = zbf ? 0xFFFF0000u : ~0u;
    float v[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      int wi;
      if constexpr (kI4) {
        const uint32_t nib = (R.w[e >> 3] >> (4 * (e & 7))) & 15u;
        wi = kSigned ? (int)(nib ^ 8u) - 8 : (int)nib;
      } else {
        const uint32_t byte = (R.w[e >> 2] >> (8 * (e & 3))) & 255u;
        wi = kSigned ? (int)(int8_t)byte : (int)byte;
      }
      const float wf = a.nf4 ? nf4[(uint32_t)wi & 15u] : (float)wi;
      float s, z = 0.0f;
      if constexpr (SM == kRgCols) {
        s = sbf ? __uint_as_float(e & 1 ? R.s[e >> 1] & 0xFFFF0000u : R.s[e >> 1] << 16) : __uint_as_float(R.s[e]);
        if (a.zp)
          z = zbf ? __uint_as_float(e & 1 ? R.z[e >> 1] & 0xFFFF0000u : R.z[e >> 1] << 16) : __uint_as_float(R.z[e]);
      } else if constexpr (SM == kRgBlk) {
        s = e < jsplit ? __uint_as_float((R.s[0] << R.ssh[0]) & smask) : __uint_as_float((R.s[1] << R.ssh[1]) & smask);
        if (a.zp)
          z = e < jsplit ? __uint_as_float((R.z[0] << R.zsh[0]) & zmask) : __uint_as_float((R.z[1] << R.zsh[1]) & zmask);
      } else {
        s = __uint_as_float((R.s[e] << R.ssh[e]) & smask);
        if (a.zp) z = __uint_as_float((R.z[e] << R.zsh[e]) & zmask);
      }
      const float ws = mul_rn(wf, s);
      v[e] = ok ? (a.zp ? add_rn(ws, z) : ws) : 0.0f;
    }
    char* bp = Bs + wrow * kRgBS + (16 * (t & 7)) * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) *(f32x4_t*)(bp + 16 * q) = f32x4_t{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) acc[i][jj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int buf) __attribute__((always_inline)) {
    const char* As = sm[buf];
    const char* Bs = sm[buf] + kRgABytes;
    float av[4][8], bv[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const char* pa = As + (wm * 64 + 16 * i + r) * kRgAS + g * 32;
      const f32x4_t lo = *(const f32x4_t*)pa, hi = *(const f32x4_t*)(pa + 16);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        av[i][e] = lo[e];
        av[i][4 + e] = hi[e];
      }
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int s = 0; s < 8; ++s) bv[jj][s] = *(const float*)(Bs + (8 * g + s) * kRgBS + (wn * 64 + 16 * jj + r) * 4);
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i][s], bv[jj][s], acc[i][jj], 0, 0, 0);
  };

  const int nkb = (K + kRgBK - 1) / kRgBK;
  Regs R;
  gload(0, R);
  __syncthreads();  // the NF4 table is written
  lstore(0, R, 0);
  __syncthreads();
#pragma unroll 1
  for (int kb = 0; kb < nkb; ++kb) {
    const bool more = kb + 1 < nkb;
    if (more) gload(kb + 1, R);
    compute(kb & 1);
    if (more) lstore(kb + 1, R, (kb + 1) & 1);
    __syncthreads();
  }

  // Epilogue: the tile goes through LDS (the buffers are free after the loop's last barrier),
  // then every thread takes outputs in row-major order: bias (added after the sum), the reference
  // activation, the output dtype.  One rolled loop, so the activation code is there once.
  constexpr int kCS = kRgBN * 4 + 16;  // LDS bytes per tile row
  static_assert(kRgBM * kCS <= 2 * kRgBuf, "the output tile fits the LDS buffers");
  char* Cs = sm[0];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *(float*)(Cs + (wm * 64 + 16 * i + 4 * g + e) * kCS + (wn * 64 + 16 * jj + r) * 4) = acc[i][jj][e];
  __syncthreads();
#pragma unroll 1
  for (int idx = t; idx < kRgBM * kRgBN; idx += kRgThreads) {
    const int row = idx / kRgBN, col = idx % kRgBN;
    const int m = m0 + row, n = n0 + col;
    if (m >= M || n >= N) continue;
    const float acc_v = *(const float*)(Cs + row * kCS + col * 4);
    const float y = a.bias ? add_rn(rg_load(a.bias, n, a.b_dt), acc_v) : acc_v;
    store_f(a.out, (int64_t)m * N + n, a.x_dt, act_ref(y, a.act));
  }
}

int rg_mode(const QDenseDesc& d) {
  if (d.block_axis == 0) return kRgCols;
  return d.block_size >= 16 ? kRgBlk : kRgAny;
}

template <int WDT, bool PLAIN>
void rg_dispatch(int mode, const RefGemmArgs& ra, int grid, hipStream_t st) {
  switch (mode) {
    case kRgCols: dispatch(qdense_refgemm_kernel<WDT, kRgCols, PLAIN>, grid, kRgThreads, 0, st, ra); break;
    case kRgBlk: dispatch(qdense_refgemm_kernel<WDT, kRgBlk, PLAIN>, grid, kRgThreads, 0, st, ra); break;
    default: dispatch(qdense_refgemm_kernel<WDT, kRgAny, PLAIN>, grid, kRgThreads, 0, st, ra); break;
  }
}

template <int WDT>
void rg_dispatch(int mode, bool plain, const RefGemmArgs& ra, int grid, hipStream_t st) {
  if (plain)
    rg_dispatch<WDT, true>(mode, ra, grid, st);
  else
    rg_dispatch<WDT, false>(mode, ra, grid, st);
}

}  // namespace

bool qdense_refgemm_fits(const QDenseDesc& d) {
  auto aligned = [](const void* p, size_t al) { return ((uintptr_t)p % al) == 0; };
  const bool xbf = d.x_dt == MX_DTYPE_BFLOAT16;
  const bool packed = dtype_is_packed(d.w_dt);
  if (!(d.scheme == MX_QUANT_LINEAR || d.scheme == MX_QUANT_NF4)) return false;
  if (!(d.x_dt == MX_DTYPE_FLOAT32 || xbf) || d.M < 1 || d.K < 8 || d.N < 16 || d.N % 16 != 0) return false;
  if (d.K % (xbf ? 8 : 4) != 0 || !aligned(d.x, 16) || !aligned(d.w, packed ? 8 : 16)) return false;
  if (d.M >= (int64_t)1 << 30 || d.K >= (int64_t)1 << 30 || d.N >= (int64_t)1 << 30) return false;
  if (d.block_axis == 0) {
    // 16 consecutive scales of a row: 16-byte loads.
    if (!aligned(d.scale, 16) || (d.zp && !aligned(d.zp, 16))) return false;
  }
  return true;
}

int qdense_refgemm_run(mx_backend* b, const QDenseDesc& d, const char* name) {
  RefGemmArgs ra{};
  ra.x = d.x;
  ra.w = (const uint8_t*)d.w;
  ra.scale = d.scale;
  ra.zp = d.zp;
  ra.bias = d.bias;
  ra.out = d.out;
  ra.M = (int)d.M;
  ra.K = (int)d.K;
  ra.N = (int)d.N;
  ra.x_dt = d.x_dt;
  ra.s_dt = d.s_dt;
  ra.zp_dt = d.zp ? d.zp_dt : MX_DTYPE_FLOAT32;
  ra.b_dt = d.b_dt;
  ra.act = d.act;
  ra.nf4 = d.scheme == MX_QUANT_NF4 ? 1 : 0;
  ra.B = (int)std::min<int64_t>(d.block_size, d.block_axis == 0 ? d.K : d.N);
  ra.nb = (int)((d.N + ra.B - 1) / ra.B);
  ra.tiles_n = (int)((d.N + kRgBN - 1) / kRgBN);
  const int64_t tiles = ((d.M + kRgBM - 1) / kRgBM) * ra.tiles_n;
  if (tiles >= (int64_t)1 << 28)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: M=%lld too large", (long long)d.M);
  ra.tiles = (int)tiles;
  ra.per_xcd = (int)((tiles + 7) / 8);
  const int grid = 8 * ra.per_xcd;
  const int mode = rg_mode(d);
  const bool plain = d.x_dt == MX_DTYPE_FLOAT32 && !d.zp && d.scheme == MX_QUANT_LINEAR;
  hipStream_t st = b->stream;
  return launch(b, name, [&] {
    switch (d.w_dt) {
      case MX_DTYPE_INT8: rg_dispatch<MX_DTYPE_INT8>(mode, plain, ra, grid, st); break;
      case MX_DTYPE_UINT8: rg_dispatch<MX_DTYPE_UINT8>(mode, plain, ra, grid, st); break;
      case MX_DTYPE_INT4: rg_dispatch<MX_DTYPE_INT4>(mode, plain, ra, grid, st); break;
      default: rg_dispatch<MX_DTYPE_UINT4>(mode, plain, ra, grid, st); break;
    }
  });
}

}  // namespace mx
