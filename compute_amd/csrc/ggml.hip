// GGML block formats on gfx950: FusedQuantizedDense with weights [N, bytesPerRow] in Q4_0, Q8_0,
// IQ4_NL, Q4_K or Q6_K blocks (K-contiguous rows), and QuantizedEmbeddingLookup.
//
// Reference semantics: quantizedDenseGGML (internal/gobackend/fusedops/quantizeddense_ggml.go:
// 103-130): per output, the row dequantised to f32 (dequantXXXRow, :158-302), dotted with x in k
// order, then the bias added, then the activation epilogue (fusedops/dense.go:176-205); x and
// the output are f32 (:58-60).  execQuantizedEmbeddingLookup (fusedops/quantizeddense.go:455-499):
// each index selects a row, dequantised to f32; an index outside [0, vocab) is an error.
//
// Kernels:
//   ggml_dense_exact — one output column per thread, k in order, every value dequantised and
//                      every product and sum rounded as the reference rounds them: bit-identical
//                      to the reference's f32 result.
//   ggml_gemv<T, MR, CH, WV> — M <= 4 rows (decode), 8 or 16 waves: a wave per output column at a
//                      time, the column's row of blocks staged through LDS with 16-byte loads (a
//                      row is contiguous), x in
//                      LDS as [m][32-value unit][36] (padded so that the 16 lanes of a 16-byte
//                      read hit distinct banks).  Each lane takes 32-value units: their integer
//                      codes times x are summed in f32 and the unit's scale (and min) applied
//                      once, then the wave adds its lanes in a fixed tree.  f32 FMAs on the VALU:
//                      x is f32 by contract, and bf16 matrix-core operands would not keep the
//                      f32 accumulation bound.
//   ggml_dequant_f32 — past 20 rows: a workgroup per row dequantises it (staged in LDS) to f32,
//                      eight values per thread, for the f32 DotGeneral; ggml_epilogue then adds
//                      the bias and applies the activation in place.
//   ggml_embed       — one thread per output value (the reference's arithmetic, bit-identical);
//                      indices of any integer dtype, bad indices reported after the launch.
// Plans: up to 4 rows the GEMV; problems of at most 2^24 multiply-adds the exact kernel; up to 20
// rows the GEMV once per group of four rows; past that the rows dequantised once to f32 [N, K]
// (each value exactly as the reference forms it), contracted on the f32 matrix cores (DotGeneral
// with a transposed right-hand side) and the bias and activation applied in place, within the f32
// accumulation bound of the reference's sum.  The exact backend option selects the exact kernel;
// the allocation-free entry point never takes the dequantised path.
#include <algorithm>
#include <cstring>

#include "device_common.h"
#include "mxrt_internal.h"

namespace mx {

typedef float f32x4_v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));

__host__ __device__ constexpr int ggml_vpb(int t) {
  return (t == MX_GGML_Q4_0 || t == MX_GGML_Q8_0 || t == MX_GGML_IQ4_NL) ? 32
         : (t == MX_GGML_Q4_K || t == MX_GGML_Q6_K)                        ? 256
                                                                            : 0;
}
__host__ __device__ constexpr int ggml_bpb(int t) {
  return (t == MX_GGML_Q4_0 || t == MX_GGML_IQ4_NL) ? 18
         : t == MX_GGML_Q8_0                        ? 34
         : t == MX_GGML_Q4_K                        ? 144
         : t == MX_GGML_Q6_K                        ? 210
                                                    : 0;
}

int ggml_block_geometry(int type, int* vpb, int* bpb) {
  *vpb = ggml_vpb(type);
  *bpb = ggml_bpb(type);
  return *vpb ? MX_OK : set_error(MX_ERR_NOT_IMPLEMENTED, "GGML type %d not supported in fused path", type);
}

// Float16.Float32 (dtypes/float16/float16.go:17-60) on the bit pattern: exact, NaN payload kept.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t mant = h & 0x3FFu;
  uint32_t bits;
  if (e == 0x1Fu) {
    bits = sign | 0x7F800000u | (mant << 13);
  } else if (e == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      const int sh = __clz(mant) - 21;  // moves the leading one to bit 10
      mant = (mant << sh) & 0x3FFu;
      bits = sign | ((uint32_t)(1 - sh - 15 + 127) << 23) | (mant << 13);
    }
  } else {
    bits = sign | ((e + 112u) << 23) | (mant << 13);
  }
  return __uint_as_float(bits);
}

__device__ __forceinline__ float f16_at(const uint8_t* p) { return f16_bits_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

// compute.IQ4NLLookupTable (fused_ops.go:127-130).
__constant__ static const float kIQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                              1,    13,   25,  38,  53,  69,  89,  113};

// getScaleMinK4 (quantizeddense_ggml.go:229-239).
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* s, uint32_t* sc, uint32_t* m) {
  if (j < 4) {
    *sc = s[j] & 63u;
    *m = s[j + 4] & 63u;
  } else {
    *sc = (s[j + 4] & 0xFu) | ((uint32_t)(s[j - 4] >> 6) << 4);
    *m = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
  }
}

// Value i of a block, with the reference's f32 operations (dequantXXXRow).
__device__ __forceinline__ float ggml_value(int t, const uint8_t* blk, int i) {
  switch (t) {
    case MX_GGML_Q8_0:
      return mul_rn(f16_at(blk), (float)(int8_t)blk[2 + i]);
    case MX_GGML_Q4_0: {
      const uint32_t b = blk[2 + (i & 15)];
      return mul_rn(f16_at(blk), (float)((int)(i < 16 ? b & 15u : b >> 4) - 8));
    }
    case MX_GGML_IQ4_NL: {
      const uint32_t b = blk[2 + (i & 15)];
      return mul_rn(f16_at(blk), kIQ4NL[i < 16 ? b & 15u : b >> 4]);
    }
    case MX_GGML_Q4_K: {
      const int chunk = i >> 6, w = i & 63, j = 2 * chunk + (w >> 5), l = w & 31;
      uint32_t sc, m;
      scale_min_k4(j, blk + 4, &sc, &m);
      const uint32_t b = blk[16 + 32 * chunk + l];
      const float d1 = mul_rn(f16_at(blk), (float)sc), min1 = mul_rn(f16_at(blk + 2), (float)m);
      return add_rn(mul_rn(d1, (float)(w < 32 ? b & 15u : b >> 4)), -min1);
    }
    default: {  // MX_GGML_Q6_K
      const int h = i >> 7, r = i & 127, j = r >> 5, l = r & 31;
      const uint32_t qlb = blk[64 * h + 32 * (j & 1) + l];
      const uint32_t nib = (j >> 1) ? qlb >> 4 : qlb & 15u;
      const uint32_t hi2 = (blk[128 + 32 * h + l] >> (2 * j)) & 3u;
      const int q = (int)(nib | (hi2 << 4)) - 32;
      const int sc = (int8_t)blk[192 + 8 * h + 2 * j + (l >> 4)];
      return mul_rn(mul_rn(f16_at(blk + 208), (float)sc), (float)q);
    }
  }
}

// =============================================================================================
// Reference-order dense kernel.
// =============================================================================================
constexpr int kGxThreads = 256;
constexpr int kGxRows = 8;

__global__ __launch_bounds__(kGxThreads) void ggml_dense_exact_kernel(GgmlDesc d) {
  const int64_t n = (int64_t)blockIdx.x * kGxThreads + threadIdx.x;
  const int64_t m0 = (int64_t)blockIdx.y * kGxRows;
  if (n >= d.N) return;
  const int rows = (int)min<int64_t>(kGxRows, d.M - m0);
  const int vpb = ggml_vpb(d.type), bpb = ggml_bpb(d.type);
  const uint8_t* row = d.w + n * d.bpr;
  float acc[kGxRows];
#pragma unroll
  for (int r = 0; r < kGxRows; ++r) acc[r] = 0.0f;
  for (int64_t k = 0; k < d.K; ++k) {
    const float wv = ggml_value(d.type, row + (k / vpb) * bpb, (int)(k % vpb));
#pragma unroll
    for (int r = 0; r < kGxRows; ++r)
      if (r < rows) acc[r] = add_rn(acc[r], mul_rn(d.x[(m0 + r) * d.K + k], wv));
  }
#pragma unroll
  for (int r = 0; r < kGxRows; ++r)
    if (r < rows) {
      float v = acc[r];
      if (d.bias) v = add_rn(v, d.bias[n]);
      d.out[(m0 + r) * d.N + n] = act_ref(v, d.act);
    }
}

// =============================================================================================
// Decode GEMV.
// =============================================================================================
// Waves per workgroup: 16 (one workgroup per CU, x staged once per CU) where the kernel stays
// within 128 registers (M = 1, and M = 2 with rows of up to 4 chunks per lane), else 8.
constexpr int kGvWavesMax = 16;
constexpr int kGvPad = 36;  // floats per 32-value unit of x in LDS
constexpr int kGvXB = 4;    // 16-byte x loads per thread in flight while staging

// Four bytes of LDS at a 2-byte-aligned address.
__device__ __forceinline__ uint32_t lds_dword2(const uint8_t* p) {
  return (uint32_t)*(const uint16_t*)p | ((uint32_t)*(const uint16_t*)(p + 2) << 16);
}

// IQ4_NL table entries of four nibbles (one per byte of q), as four signed bytes: two byte
// permutes over the 16-byte table (as int8), the high half chosen where bit 3 is set.
__device__ __forceinline__ uint32_t iq4nl_bytes(uint32_t q) {
  constexpr uint32_t T0 = 0xBFAD9881u, T1 = 0xF6EADDCFu, T2 = 0x26190D01u, T3 = 0x71594535u;
  const uint32_t sel = q & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel), hi = __builtin_amdgcn_perm(T3, T2, sel);
  const uint32_t m = ((q >> 3) & 0x01010101u) * 0xFFu;
  return (hi & m) | (lo & ~m);
}

// Sum over one 32-value unit u of the row (starting at `row` in LDS) of x[m][32u + l] * w, for
// each of the MR rows of x (xu[m] points at the unit in LDS, sx[m] is the unit's sum of x).  The
// integer codes are converted four at a time (byte converts); a constant offset (Q4_0's -8,
// Q4_K's min) is applied through sx.
template <int T, int MR>
__device__ __forceinline__ void ggml_unit(const uint8_t* row, int u, const float* const (&xu)[MR], const float (&sx)[MR],
                                          float (&acc)[MR]) {
  auto xv = [&](int m, int l) { return xu[m][l]; };
  // s[m] += sum over the four bytes of `v` (unsigned codes) of x[m][l0 + b] * byte_b.
  auto fma4u = [&](uint32_t v, int l0, float (&s)[MR]) {
    const float q0 = (float)(v & 0xFFu), q1 = (float)((v >> 8) & 0xFFu);  // v_cvt_f32_ubyteN
    const float q2 = (float)((v >> 16) & 0xFFu), q3 = (float)(v >> 24);
#pragma unroll
    for (int m = 0; m < MR; ++m)
      s[m] = fmaf(xv(m, l0 + 3), q3, fmaf(xv(m, l0 + 2), q2, fmaf(xv(m, l0 + 1), q1, fmaf(xv(m, l0), q0, s[m]))));
  };
  auto fma4s = [&](uint32_t v, int l0, float (&s)[MR]) {  // signed bytes
    const float q0 = (float)(int8_t)v, q1 = (float)(int8_t)(v >> 8);
    const float q2 = (float)(int8_t)(v >> 16), q3 = (float)(int8_t)(v >> 24);
#pragma unroll
    for (int m = 0; m < MR; ++m)
      s[m] = fmaf(xv(m, l0 + 3), q3, fmaf(xv(m, l0 + 2), q2, fmaf(xv(m, l0 + 1), q1, fmaf(xv(m, l0), q0, s[m]))));
  };
  float s[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) s[m] = 0.0f;
  if constexpr (T == MX_GGML_Q4_0 || T == MX_GGML_IQ4_NL) {
    const uint8_t* blk = row + 18 * u;
    const float d = f16_at(blk);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = lds_dword2(blk + 2 + 4 * i);
      const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
      if constexpr (T == MX_GGML_Q4_0) {
        fma4u(lo, 4 * i, s);
        fma4u(hi, 16 + 4 * i, s);
      } else {
        fma4s(iq4nl_bytes(lo), 4 * i, s);
        fma4s(iq4nl_bytes(hi), 16 + 4 * i, s);
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = fmaf(d, T == MX_GGML_Q4_0 ? fmaf(-8.0f, sx[m], s[m]) : s[m], acc[m]);
  } else if constexpr (T == MX_GGML_Q8_0) {
    const uint8_t* blk = row + 34 * u;
    const float d = f16_at(blk);
#pragma unroll
    for (int i = 0; i < 8; ++i) fma4s(lds_dword2(blk + 2 + 4 * i), 4 * i, s);
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = fmaf(d, s[m], acc[m]);
  } else if constexpr (T == MX_GGML_Q4_K) {
    const int jj = u & 7;
    const uint8_t* blk = row + 144 * (u >> 3);
    uint32_t sc, mn;
    scale_min_k4(jj, blk + 4, &sc, &mn);
    const float a = f16_at(blk) * (float)sc, b = f16_at(blk + 2) * (float)mn;
    const uint8_t* qs = blk + 16 + 32 * (jj >> 1);
    const int sh = 4 * (jj & 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) fma4u((lds_dword2(qs + 4 * i) >> sh) & 0x0F0F0F0Fu, 4 * i, s);
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = fmaf(a, s[m], fmaf(-b, sx[m], acc[m]));
  } else {  // MX_GGML_Q6_K: unit = quarter j of half h of a super-block
    const int v = u & 7, h = v >> 2, j = v & 3;
    const uint8_t* blk = row + 210 * (u >> 3);
    const float d = f16_at(blk + 208);
    const uint8_t* ql = blk + 64 * h + 32 * (j & 1);
    const uint8_t* qh = blk + 128 + 32 * h;
    const int nsh = 4 * (j >> 1), hsh = 2 * j;
    const float sc0 = d * (float)(int8_t)blk[192 + 8 * h + 2 * j], sc1 = d * (float)(int8_t)blk[192 + 8 * h + 2 * j + 1];
    float s1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) s1[m] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t q = ((lds_dword2(ql + 4 * i) >> nsh) & 0x0F0F0F0Fu) | (((lds_dword2(qh + 4 * i) >> hsh) & 0x03030303u) << 4);
      // Codes 0..63 stand for q - 32, the 6-bit two's complement value of q ^ 32: shifted into
      // the top of each byte it reads as the signed byte 4 * (q - 32) (no carries between bytes).
      fma4s((q ^ 0x20202020u) << 2, 4 * i, i < 4 ? s : s1);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = fmaf(0.25f * sc0, s[m], fmaf(0.25f * sc1, s1[m], acc[m]));
  }
}

// CH: 16-byte chunks of a row per lane (the row, with its alignment skew, is at most 64*CH chunks).
template <int T, int MR, int CH, int WV>
__global__ __launch_bounds__(64 * WV) void ggml_gemv_kernel(GgmlDesc d) {
  constexpr int kGvWaves = WV, kGvThreads = 64 * WV;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int kRowBytes = 64 * CH * 16;
  const int K = (int)d.K, units = K >> 5;
  float* xs = (float*)lds;                                             // [MR][units][kGvPad]
  uint8_t* rows = lds + (size_t)MR * units * kGvPad * sizeof(float);   // [waves][kRowBytes]
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  uint8_t* rb = rows + (size_t)wave * kRowBytes;
  // The weights are read in whole 16-byte units from a 16-byte-aligned base: the buffer's range
  // is its size rounded up to 16 (a partially valid unit must come back whole; the bytes past
  // the end lie in the same allocation granule, 256 bytes or more) and units beyond it read 0.
  // A row (or its K segment: bpr bytes from row_off) starts r * rstride + row_off bytes in.
  const int64_t rstride = d.row_stride ? d.row_stride : d.bpr;
  const int64_t ldx = d.ldx ? d.ldx : d.K;
  const int64_t total = (d.N * rstride + 15) & ~(int64_t)15;
  const __amdgpu_buffer_rsrc_t wrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(d.w), (short)0, (int)total, 0x00020000);
  // A row is loaded into registers one row ahead (16-byte loads from the aligned address at or
  // below its start; the row then begins `skew` bytes into the staging buffer), so its loads
  // travel while the previous row is computed.  Chunks past the row's end are given an offset
  // past the buffer's range: they read 0 without a memory access.  (Two rows ahead took 16 more
  // registers, past the 128 that keep two workgroups on a CU, and measured slower.)
  u32x4_v pre[CH];
  auto issue = [&](int64_t row, u32x4_v (&dst)[CH]) {
    const int64_t r = min(row, d.N - 1);
    const int64_t rs = r * rstride + d.row_off;
    const uint32_t a0 = (uint32_t)(rs & ~(int64_t)15), end = (uint32_t)(rs + d.bpr);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const uint32_t off = a0 + 16u * (lane + 64 * i);
      dst[i] = __builtin_amdgcn_raw_buffer_load_b128(wrs, off < end ? off : 0x7FFFFFF0u, 0, 0);
    }
  };
  // Each workgroup takes a contiguous run of rows, N / grid of them (one more for the first
  // N % grid), so that no CU has more than one row above the average; its waves take every
  // WV-th row of the run.
  const int64_t r1 = (int64_t)(blockIdx.x + 1) * d.N / gridDim.x;
  const int64_t stride = kGvWaves;
  int64_t n = (int64_t)blockIdx.x * d.N / gridDim.x + wave;
  if (n < r1) issue(n, pre);  // before staging x: the first row travels meanwhile
  // x staged as [MR][units][kGvPad] floats with 16-byte loads, kGvXB of them issued before their
  // stores (K % 32 == 0, ldx % 4 == 0, x 16-byte aligned).
  {
    const int q4 = K / 4;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float4* xr = reinterpret_cast<const float4*>(d.x + m * ldx);
      for (int base = t; base < q4; base += kGvXB * kGvThreads) {
        float4 v[kGvXB];
#pragma unroll
        for (int j = 0; j < kGvXB; ++j)  // unconditional (clamped) so that they stay in registers
          v[j] = xr[min(base + j * kGvThreads, q4 - 1)];
#pragma unroll
        for (int j = 0; j < kGvXB; ++j) {
          const int i = base + j * kGvThreads;
          if (i < q4) {
            const int k = 4 * i;
            *reinterpret_cast<float4*>(xs + (m * units + (k >> 5)) * kGvPad + (k & 31)) = v[j];
          }
        }
      }
    }
  }
  __syncthreads();
  // Each unit's sum of x, kept in the unit's padding (slot 32), in a fixed order (four partial
  // sums over the unit's 16-byte chunks, then added in order).
  for (int i = t; i < MR * units; i += kGvThreads) {
    float* xu = xs + (size_t)i * kGvPad;
    float4 a = reinterpret_cast<const float4*>(xu)[0];
#pragma unroll
    for (int c = 1; c < 8; ++c) {
      const float4 v = reinterpret_cast<const float4*>(xu)[c];
      a.x += v.x;
      a.y += v.y;
      a.z += v.z;
      a.w += v.w;
    }
    xu[32] = (a.x + a.y) + (a.z + a.w);
  }
  __syncthreads();

  for (; n < r1; n += stride) {
#pragma unroll
    for (int i = 0; i < CH; ++i) *(u32x4_v*)(rb + 16 * (lane + 64 * i)) = pre[i];
    if (n + stride < r1) issue(n + stride, pre);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    const uint8_t* row = rb + (int)((n * rstride + d.row_off) & 15);
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
    for (int u = lane; u < units; u += 64) {
      const float* xu[MR];
      float sx[MR];
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        xu[m] = xs + (size_t)(m * units + u) * kGvPad;
        sx[m] = xu[m][32];
      }
      ggml_unit<T, MR>(row, u, xu, sx, acc);
    }
    // Lanes in a fixed tree.
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) acc[m] += __shfl_xor(acc[m], off, 64);
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        float v = acc[m];
        float* o = d.out + (size_t)m * d.N + n;
        if (d.accumulate) v = add_rn(*o, v);  // the earlier K segments' sum first
        if (d.epilogue) {
          if (d.bias) v = add_rn(v, d.bias[n]);
          v = act_ref(v, d.act);
        }
        *o = v;
      }
    }
    // Every lane's reads of the row are done before the next row is staged over it.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
  }
}

// Chunks per lane (2, 4 or 8), waves per workgroup (8 or 16) and LDS of the GEMV for these
// sizes, or 0 if it does not apply.
static size_t ggml_gemv_lds(const GgmlDesc& d, int* ch, int* waves) {
  const int64_t rstride = d.row_stride ? d.row_stride : d.bpr, ldx = d.ldx ? d.ldx : d.K;
  if (d.M < 1 || d.M > 4 || d.K % 32 != 0 || d.K > (1 << 20) || d.N * rstride + 16 >= ((int64_t)1 << 31) ||
      ldx % 4 != 0 || (uintptr_t)d.w % 16 != 0 || (uintptr_t)d.x % 16 != 0)
    return 0;
  const int64_t chunks = (d.bpr + 15 + 15) / 16;  // worst-case skew included
  int c = 2;
  while (c < 8 && 64 * c < chunks) c *= 2;
  if (64 * c < chunks) return 0;
  const size_t xb = (size_t)d.M * (d.K / 32) * kGvPad * sizeof(float);
  int wv = d.M == 1 || (d.M == 2 && c <= 4) ? kGvWavesMax : 8;
  if (xb + (size_t)wv * 64 * c * 16 > 150 * 1024) wv = 8;
  const size_t bytes = xb + (size_t)wv * 64 * c * 16;
  if (bytes > 150 * 1024) return 0;
  *ch = c;
  *waves = wv;
  return bytes;
}

template <int T, int CH>
static void launch_gemv_ch(const GgmlDesc& d, int grid, size_t lds, int waves, hipStream_t st) {
  const bool w16 = waves == 16;
  switch (d.M) {
    case 1:
      w16 ? dispatch(ggml_gemv_kernel<T, 1, CH, 16>, grid, 1024, lds, st, d)
          : dispatch(ggml_gemv_kernel<T, 1, CH, 8>, grid, 512, lds, st, d);
      break;
    case 2:
      w16 ? dispatch(ggml_gemv_kernel<T, 2, CH, 16>, grid, 1024, lds, st, d)
          : dispatch(ggml_gemv_kernel<T, 2, CH, 8>, grid, 512, lds, st, d);
      break;
    case 3: dispatch(ggml_gemv_kernel<T, 3, CH, 8>, grid, 512, lds, st, d); break;
    default: dispatch(ggml_gemv_kernel<T, 4, CH, 8>, grid, 512, lds, st, d); break;
  }
}

template <int T>
static void launch_gemv_t(const GgmlDesc& d, int grid, size_t lds, int ch, int waves, hipStream_t st) {
  if (ch == 2)
    launch_gemv_ch<T, 2>(d, grid, lds, waves, st);
  else if (ch == 4)
    launch_gemv_ch<T, 4>(d, grid, lds, waves, st);
  else
    launch_gemv_ch<T, 8>(d, grid, lds, waves, st);
}


// Prefill: the rows dequantised to f32 [N, K], each value as the reference forms it (the
// arithmetic of ggml_value, the type fixed at compile time).  A workgroup per row at a
// time: the row's bytes staged in LDS with coalesced 2-byte loads (every block size is even),
// then eight consecutive values (one block's) per thread decoded from LDS and written as two
// 16-byte stores.  Rows of up to kDqRowBytes bytes (dynamic LDS of the row's size).
constexpr int kDqRowBytes = 64 * 1024;

// Values i .. i+7 of a block (i a multiple of 8), as ggml_value forms each one, with what the
// eight share (the block scale, a K-quant sub-block's scale and minimum) formed once.
template <int T>
__device__ __forceinline__ void ggml_values8(const uint8_t* blk, int i, float* v) {
  if constexpr (T == MX_GGML_Q8_0) {
    const float d = f16_at(blk);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = mul_rn(d, (float)(int8_t)blk[2 + i + e]);
  } else if constexpr (T == MX_GGML_Q4_0 || T == MX_GGML_IQ4_NL) {
    const float d = f16_at(blk);
    const uint8_t* q = blk + 2 + (i & 15);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t nib = i < 16 ? q[e] & 15u : (uint32_t)q[e] >> 4;
      v[e] = T == MX_GGML_Q4_0 ? mul_rn(d, (float)((int)nib - 8)) : mul_rn(d, kIQ4NL[nib]);
    }
  } else if constexpr (T == MX_GGML_Q4_K) {
    const int chunk = i >> 6, w = i & 63, j = 2 * chunk + (w >> 5);
    uint32_t sc, m;
    scale_min_k4(j, blk + 4, &sc, &m);
    const float d1 = mul_rn(f16_at(blk), (float)sc), min1 = mul_rn(f16_at(blk + 2), (float)m);
    const uint8_t* q = blk + 16 + 32 * chunk + (w & 31);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = add_rn(mul_rn(d1, (float)(w < 32 ? q[e] & 15u : (uint32_t)q[e] >> 4)), -min1);
  } else {  // MX_GGML_Q6_K
    const int h = i >> 7, r = i & 127, j = r >> 5, l = r & 31;
    const float ds = mul_rn(f16_at(blk + 208), (float)(int)(int8_t)blk[192 + 8 * h + 2 * j + (l >> 4)]);
    const uint8_t* ql = blk + 64 * h + 32 * (j & 1) + l;
    const uint8_t* qh = blk + 128 + 32 * h + l;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t nib = (j >> 1) ? (uint32_t)ql[e] >> 4 : ql[e] & 15u;
      const uint32_t hi2 = ((uint32_t)qh[e] >> (2 * j)) & 3u;
      v[e] = mul_rn(ds, (float)((int)(nib | (hi2 << 4)) - 32));
    }
  }
}

template <int T>
__global__ __launch_bounds__(256) void ggml_dequant_f32_kernel(GgmlDesc d, float* __restrict__ wt) {
  constexpr int vpb = T == MX_GGML_Q4_K || T == MX_GGML_Q6_K ? 256 : 32;
  constexpr int vsh = vpb == 256 ? 8 : 5;
  extern __shared__ __align__(16) uint16_t rs[];
  const uint8_t* rb = reinterpret_cast<const uint8_t*>(rs);
  const int bpb = ggml_bpb(T);
  const int K8 = (int)(d.K / 8), H = (int)(d.bpr / 2);
  for (int64_t n = blockIdx.x; n < d.N; n += gridDim.x) {
    const uint16_t* row = reinterpret_cast<const uint16_t*>(d.w + n * d.bpr);
    for (int h = threadIdx.x; h < H; h += blockDim.x) rs[h] = row[h];
    __syncthreads();
    float4* out = reinterpret_cast<float4*>(wt + n * d.K);
    for (int j = threadIdx.x; j < K8; j += blockDim.x) {
      const int k = 8 * j;
      const uint8_t* blk = rb + (k >> vsh) * bpb;
      const int i = k & (vpb - 1);
      float v[8];
      ggml_values8<T>(blk, i, v);
      out[2 * j] = make_float4(v[0], v[1], v[2], v[3]);
      out[2 * j + 1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();
  }
}

// In place on the f32 sums: the bias added after the sum (the reference's order), then the
// reference activation.
__global__ void ggml_epilogue_kernel(float* __restrict__ y, const float* __restrict__ bias, int act, int64_t M,
                                     int64_t N) {
  const int64_t total = M * N;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    float v = y[i];
    if (bias) v = add_rn(v, bias[i % N]);
    y[i] = act_ref(v, act);
  }
}

// The K segment of the decode GEMV for these rows: the whole row where it fits (row bytes up to
// 8 chunks per lane, the rows of x within the LDS), else the longest of ceil(blocks / s) blocks,
// s = 2, 3, ... 64, that fits; 0 if none does.  Segment j runs as its own launch over bytes
// j * seg of every row and the matching x columns, adding its sums to the output the earlier
// segments wrote (in segment order); the last applies the bias and the activation.  Without it
// rows past 8 KB, or longer rows of x than the LDS holds (two rows at K = 14336), took the
// dequantise + matrix-core path: 150-160 us per call for one or two rows of [14336] x 4096 rows
// against about 20 us for the GEMV.
static int64_t ggml_gemv_kseg(const GgmlDesc& d) {
  int ch, wv;
  if (ggml_gemv_lds(d, &ch, &wv)) return d.K;
  const int vpb = ggml_vpb(d.type), bpb = ggml_bpb(d.type);
  if (!vpb || d.K % vpb != 0) return 0;
  const int64_t blocks = d.K / vpb;
  for (int64_t sg = 2; sg <= 64 && sg <= blocks; ++sg) {
    const int64_t nb = (blocks + sg - 1) / sg;
    GgmlDesc g = d;
    g.K = nb * vpb;
    g.bpr = nb * bpb;
    g.ldx = d.K;
    g.row_stride = d.bpr;
    if (ggml_gemv_lds(g, &ch, &wv)) return g.K;
  }
  return 0;
}

enum class GPlan { kEmpty, kGemv, kDequant, kExact };

static GPlan ggml_plan(const mx_backend* b, const GgmlDesc& d) {
  if (d.M == 0 || d.N == 0) return GPlan::kEmpty;
  if (b->exact_qdense) return GPlan::kExact;
  int ch;
  int wv;
  if (d.M <= 4 && ggml_gemv_lds(d, &ch, &wv)) return GPlan::kGemv;
  // Problems this small keep the reference's order (bit-identical).
  if (d.M * d.K * d.N <= ((int64_t)1 << 24)) return GPlan::kExact;
  if (d.M <= 4 && ggml_gemv_kseg(d)) return GPlan::kGemv;  // in K segments
  GgmlDesc g4 = d;
  g4.M = 4;
  const bool gemv4 = ggml_gemv_kseg(g4) != 0;
  // The weights read once per group of four rows (about 27 us a group at [4096] x 11008 rows),
  // until one dequantisation and a matrix-core contraction (about 143 us there past 16 rows)
  // cost less; both scale with the weight bytes, so the crossover holds across shapes.
  if (d.M <= 20 && gemv4) return GPlan::kGemv;
  // The dequantised matrix is a device allocation: not for the allocation-free entry point.
  if (!b->noalloc_active && d.N * d.K * 4 <= ((int64_t)8 << 30) && d.bpr <= kDqRowBytes && d.bpr % 2 == 0 && (uintptr_t)d.w % 2 == 0 &&
      (uintptr_t)d.x % 16 == 0)
    return GPlan::kDequant;
  return gemv4 ? GPlan::kGemv : GPlan::kExact;
}

const char* ggml_plan_name(const mx_backend* b, const GgmlDesc& d) {
  switch (ggml_plan(b, d)) {
    case GPlan::kEmpty: return "empty";
    case GPlan::kGemv: return "ggml_gemv";
    case GPlan::kDequant: return "ggml_dequant_f32_mfma";
    default: return "ggml_dense_exact";
  }
}

int ggml_dense_run(mx_backend* b, const GgmlDesc& d) {
  MX_TRY(check_device(b));
  hipStream_t st = b->stream;
  switch (ggml_plan(b, d)) {
    case GPlan::kEmpty:
      return MX_OK;
    case GPlan::kGemv: {
      // Groups of up to four rows, one launch each per K segment.
      const int vpb = ggml_vpb(d.type), bpb = ggml_bpb(d.type);
      for (int64_t m0 = 0; m0 < d.M; m0 += 4) {
        GgmlDesc rows = d;
        rows.x = d.x + m0 * d.K;
        rows.out = d.out + m0 * d.N;
        rows.M = std::min<int64_t>(4, d.M - m0);
        const int64_t kseg = ggml_gemv_kseg(rows);
        if (!kseg || (kseg < d.K && !vpb)) return set_error(MX_ERR_INVALID, "internal: GGML GEMV plan without a launch");
        for (int64_t k0 = 0; k0 < d.K; k0 += kseg) {
          GgmlDesc g = rows;
          if (kseg < d.K) {
            const int64_t kl = std::min<int64_t>(kseg, d.K - k0);
            g.x = rows.x + k0;
            g.ldx = d.K;
            g.K = kl;
            g.bpr = kl / vpb * bpb;
            g.row_stride = d.bpr;
            g.row_off = k0 / vpb * bpb;
            g.accumulate = k0 > 0;
            g.epilogue = k0 + kl >= d.K;
          }
          int ch = 0;
          int waves = 8;
          const size_t lds = ggml_gemv_lds(g, &ch, &waves);
          if (!lds) return set_error(MX_ERR_INVALID, "internal: GGML GEMV plan without a launch");
          // As many workgroups as are resident at once: 16 waves per CU (four per SIMD at up to 128
          // registers), fewer where LDS runs out.
          const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(16 / waves, (int64_t)(160 * 1024) / (int64_t)lds));
          const int grid = (int)std::min<int64_t>((g.N + waves - 1) / waves, per_cu * std::max(b->num_cus, 1));
          MX_TRY(launch(b, "ggml_gemv", [&] {
            switch (g.type) {
              case MX_GGML_Q4_0: launch_gemv_t<MX_GGML_Q4_0>(g, grid, lds, ch, waves, st); break;
              case MX_GGML_Q8_0: launch_gemv_t<MX_GGML_Q8_0>(g, grid, lds, ch, waves, st); break;
              case MX_GGML_IQ4_NL: launch_gemv_t<MX_GGML_IQ4_NL>(g, grid, lds, ch, waves, st); break;
              case MX_GGML_Q4_K: launch_gemv_t<MX_GGML_Q4_K>(g, grid, lds, ch, waves, st); break;
              default: launch_gemv_t<MX_GGML_Q6_K>(g, grid, lds, ch, waves, st); break;
            }
          }));
        }
      }
      return MX_OK;
    }
    case GPlan::kDequant: {
      void* wt = nullptr;
      MX_TRY(dev_alloc(b, (size_t)(d.N * d.K) * 4, &wt));
      const int rows = (int)std::min<int64_t>(d.N, 8 * (int64_t)std::max(b->num_cus, 1));
      const size_t lds = (size_t)(d.bpr + 15) / 16 * 16;
      int rc = launch(b, "ggml_dequant_f32", [&] {
        switch (d.type) {
          case MX_GGML_Q4_0: dispatch(ggml_dequant_f32_kernel<MX_GGML_Q4_0>, rows, 256, lds, st, d, (float*)wt); break;
          case MX_GGML_Q8_0: dispatch(ggml_dequant_f32_kernel<MX_GGML_Q8_0>, rows, 256, lds, st, d, (float*)wt); break;
          case MX_GGML_IQ4_NL: dispatch(ggml_dequant_f32_kernel<MX_GGML_IQ4_NL>, rows, 256, lds, st, d, (float*)wt); break;
          case MX_GGML_Q4_K: dispatch(ggml_dequant_f32_kernel<MX_GGML_Q4_K>, rows, 256, lds, st, d, (float*)wt); break;
          default: dispatch(ggml_dequant_f32_kernel<MX_GGML_Q6_K>, rows, 256, lds, st, d, (float*)wt); break;
        }
      });
      if (rc == MX_OK) {
        DotDesc dd{};
        dd.lhs = d.x;
        dd.rhs = wt;
        dd.out = d.out;
        dd.B = 1;
        dd.M = d.M;
        dd.K = d.K;
        dd.N = d.N;
        dd.rhs_transposed = true;
        dd.in_dt = MX_DTYPE_FLOAT32;
        dd.out_dt = MX_DTYPE_FLOAT32;
        rc = dot_run(b, dd);
      }
      if (rc == MX_OK)
        rc = launch(b, "ggml_epilogue", [&] { dispatch(ggml_epilogue_kernel, 1024, 256, 0, st, d.out, d.bias, d.act, d.M, d.N); });
      dev_free(b, wt);  // stream-ordered pool: later users run after these kernels
      return rc;
    }
    default: {
      dim3 grid((unsigned)((d.N + kGxThreads - 1) / kGxThreads), (unsigned)((d.M + kGxRows - 1) / kGxRows));
      if (grid.y > 65535u) return set_error(MX_ERR_INVALID, "FusedQuantizedDense(GGML): M too large");
      return launch(b, "ggml_dense_exact", [&] { dispatch(ggml_dense_exact_kernel, grid, kGxThreads, 0, st, d); });
    }
  }
}

// =============================================================================================
// QuantizedEmbeddingLookup.
// =============================================================================================
__device__ __forceinline__ int64_t load_index(const void* p, int64_t i, int dt) {
  switch (dt) {
    case MX_DTYPE_INT8: return ((const int8_t*)p)[i];
    case MX_DTYPE_INT16: return ((const int16_t*)p)[i];
    case MX_DTYPE_INT32: return ((const int32_t*)p)[i];
    case MX_DTYPE_UINT8: return ((const uint8_t*)p)[i];
    case MX_DTYPE_UINT16: return ((const uint16_t*)p)[i];
    case MX_DTYPE_UINT32: return ((const uint32_t*)p)[i];
    case MX_DTYPE_UINT64: {
      const uint64_t v = ((const uint64_t*)p)[i];
      return v > (uint64_t)INT64_MAX ? -1 : (int64_t)v;
    }
    default: return ((const int64_t*)p)[i];
  }
}

// One thread per output value; a bad index writes nothing and records its position (the
// smallest one) in *bad, which the host reads back.
__global__ void ggml_embed_kernel(GgmlEmbedDesc e, unsigned long long* bad) {
  const int64_t total = e.n * e.K;
  const int vpb = ggml_vpb(e.type), bpb = ggml_bpb(e.type);
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < total; p += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = p / e.K, k = p - i * e.K;
    const int64_t r = load_index(e.idx, i, e.idx_dt);
    if (r < 0 || r >= e.vocab) {
      if (k == 0) atomicMin(bad, (unsigned long long)i);
      continue;
    }
    e.out[p] = ggml_value(e.type, e.data + r * e.bpr + (k / vpb) * bpb, (int)(k % vpb));
  }
}

__global__ void ggml_fill_u64(unsigned long long* p, unsigned long long v) { *p = v; }

int ggml_embed_run(mx_backend* b, const GgmlEmbedDesc& e) {
  MX_TRY(check_device(b));
  if (e.n == 0 || e.K == 0) return MX_OK;
  void* flag = nullptr;
  MX_TRY(dev_alloc(b, sizeof(unsigned long long), &flag));
  unsigned long long* bad = (unsigned long long*)flag;
  hipStream_t st = b->stream;
  const int64_t total = e.n * e.K;
  const int grid = (int)std::min<int64_t>((total + 255) / 256, 65536);
  int rc = launch(b, "ggml_embed", [&] {
    dispatch(ggml_fill_u64, 1, 1, 0, st, bad, ~0ull);
    dispatch(ggml_embed_kernel, grid, 256, 0, st, e, bad);
  });
  unsigned long long h = ~0ull;
  if (rc == MX_OK) {
    // The reference reports an out-of-range index as an error of the call, so the result of
    // the check has to be known before returning.
    if (hipMemcpyAsync(&h, bad, sizeof(h), hipMemcpyDeviceToHost, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
      rc = set_error(MX_ERR_HIP, "QuantizedEmbeddingLookup: reading the index check failed");
  }
  dev_free(b, flag);
  if (rc != MX_OK || h == ~0ull) return rc;
  // The offending value, for the message the reference gives.
  const int isz = (e.idx_dt == MX_DTYPE_INT8 || e.idx_dt == MX_DTYPE_UINT8)     ? 1
                  : (e.idx_dt == MX_DTYPE_INT16 || e.idx_dt == MX_DTYPE_UINT16) ? 2
                  : (e.idx_dt == MX_DTYPE_INT32 || e.idx_dt == MX_DTYPE_UINT32) ? 4
                                                                                : 8;
  uint8_t raw[8] = {0};
  if (hipMemcpy(raw, (const uint8_t*)e.idx + h * isz, isz, hipMemcpyDeviceToHost) != hipSuccess)
    return set_error(MX_ERR_HIP, "QuantizedEmbeddingLookup: reading the bad index failed");
  long long v = 0;
  switch (e.idx_dt) {
    case MX_DTYPE_INT8: v = *(int8_t*)raw; break;
    case MX_DTYPE_INT16: v = *(int16_t*)raw; break;
    case MX_DTYPE_INT32: v = *(int32_t*)raw; break;
    case MX_DTYPE_UINT8: v = *(uint8_t*)raw; break;
    case MX_DTYPE_UINT16: v = *(uint16_t*)raw; break;
    case MX_DTYPE_UINT32: v = *(uint32_t*)raw; break;
    default: memcpy(&v, raw, 8); break;
  }
  return set_error(MX_ERR_INVALID, "QuantizedEmbeddingLookup: index %lld out of range [0, %lld)", v, (long long)e.vocab);
}

}  // namespace mx

// =============================================================================================
// C ABI: direct embedding lookup.
// =============================================================================================
extern "C" int mx_quantized_embedding_lookup(mx_backend* b, const mx_qembed_args* a) {
  mx::clear_error();
  MX_TRY(mx::check_device(b));
  const char* op = "QuantizedEmbeddingLookup";
  if (!a) return mx::set_error(MX_ERR_INVALID, "%s: args is NULL", op);
  int vpb, bpb;
  switch (a->ggml_type) {
    case MX_GGML_Q4_0: case MX_GGML_Q8_0: case MX_GGML_IQ4_NL: case MX_GGML_Q4_K: case MX_GGML_Q6_K: break;
    default:
      return mx::set_error(MX_ERR_NOT_IMPLEMENTED, "%s: GGML type %d not supported in fused path", op, a->ggml_type);
  }
  MX_TRY(mx::ggml_block_geometry(a->ggml_type, &vpb, &bpb));
  switch (a->index_dtype) {
    case MX_DTYPE_INT8: case MX_DTYPE_INT16: case MX_DTYPE_INT32: case MX_DTYPE_INT64:
    case MX_DTYPE_UINT8: case MX_DTYPE_UINT16: case MX_DTYPE_UINT32: case MX_DTYPE_UINT64: break;
    default: return mx::set_error(MX_ERR_INVALID, "%s: indices must be integer, got %s", op, mx::dtype_name(a->index_dtype));
  }
  if (a->bytes_per_row < 0 || a->bytes_per_row % bpb != 0 || a->vocab < 0 || a->n < 0)
    return mx::set_error(MX_ERR_INVALID, "%s: bytesPerRow %lld not divisible by bytesPerBlock %d", op,
                         (long long)a->bytes_per_row, bpb);
  mx::GgmlEmbedDesc e;
  e.data = (const uint8_t*)a->data;
  e.idx = a->indices;
  e.out = (float*)a->out;
  e.vocab = a->vocab;
  e.bpr = a->bytes_per_row;
  e.K = a->bytes_per_row / bpb * vpb;
  e.n = a->n;
  e.idx_dt = a->index_dtype;
  e.type = a->ggml_type;
  if (e.n * e.K > 0 && (!e.out || !e.idx || !e.data)) return mx::set_error(MX_ERR_INVALID, "%s: NULL data pointer", op);
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  return mx::ggml_embed_run(b, e);
}
