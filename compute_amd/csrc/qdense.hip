// FusedQuantizedDense on gfx950: argument validation, kernel selection and the kernels.
//
// Reference semantics (internal/gobackend/fusedops/quantizeddense.go:616-650, Linear scheme):
//   out[m,n] = bias[n] (or 0);  for k in 0..K-1:  out[m,n] += x[m,k] * float32(w[k,n]) * s
// with s = scale[k, n/B] (reference layout, BlockAxis=1) and, with a zero point,
//   out[m,n] += x[m,k] * (float32(w[k,n]) * s + zp)
// then the activation epilogue over the whole output (fusedops/dense.go:176-205).
// NF4 replaces float32(w) with NF4Table[uint8(w) & 15] (quantizeddense.go:586-609).
//
// This backend also accepts scales blocked along K (BlockAxis=0, scale[k/B, n]): the
// per-group / per-output-channel layouts that weight-only quantized LLM checkpoints use.
//
// Kernels:
//   qdense_exact   — one output column per thread, k in order, each term rounded exactly as the
//                    reference loop rounds it: bit-identical to the reference's f32 result.
//                    Used for f32 activations and any shape/layout without a fast path.
//   gemv_dot2      — M=1, bf16 x (decode). HBM-bound: 128-bit weight loads, nibble/byte ->
//                    bf16 pairs in registers, v_dot2_f32_bf16 MACs, per-group scale applied
//                    once per wave, split-K with a deterministic last-arriver reduction.

#include <algorithm>
#include <string>

#include "device_common.h"
#include "mxrt_internal.h"

namespace mx {

// =============================================================================================
// Validation.
// =============================================================================================
static bool is_f32_or_bf16(int dt) { return dt == MX_DTYPE_FLOAT32 || dt == MX_DTYPE_BFLOAT16; }

int qdense_validate(const mx_qdense_args* a, QDenseDesc* d) {
  if (!a) return set_error(MX_ERR_INVALID, "FusedQuantizedDense: args is NULL");
  if (a->scheme == MX_QUANT_GGML)
    return set_error(MX_ERR_NOT_IMPLEMENTED, "FusedQuantizedDense: GGML block formats are not implemented");
  if (a->scheme != MX_QUANT_LINEAR && a->scheme != MX_QUANT_NF4)
    return set_error(MX_ERR_NOT_IMPLEMENTED, "FusedQuantizedDense: unknown quantization scheme %d", a->scheme);
  if (!is_f32_or_bf16(a->x_dtype))
    return set_error(MX_ERR_NOT_IMPLEMENTED, "FusedQuantizedDense: x must be Float32 or BFloat16, got %s",
                     dtype_name(a->x_dtype));
  switch (a->w_dtype) {
    case MX_DTYPE_INT8: case MX_DTYPE_UINT8: case MX_DTYPE_INT4: case MX_DTYPE_UINT4: break;
    default:
      return set_error(MX_ERR_NOT_IMPLEMENTED, "FusedQuantizedDense: unsupported weight dtype %s",
                       dtype_name(a->w_dtype));
  }
  if (!is_f32_or_bf16(a->scale_dtype))
    return set_error(MX_ERR_NOT_IMPLEMENTED, "FusedQuantizedDense: scale must be Float32 or BFloat16, got %s",
                     dtype_name(a->scale_dtype));
  if (a->zero_point && !is_f32_or_bf16(a->zero_point_dtype))
    return set_error(MX_ERR_NOT_IMPLEMENTED, "FusedQuantizedDense: zero point must be Float32 or BFloat16");
  if (a->bias && !is_f32_or_bf16(a->bias_dtype))
    return set_error(MX_ERR_NOT_IMPLEMENTED, "FusedQuantizedDense: bias must be Float32 or BFloat16");
  if (a->scheme == MX_QUANT_NF4 && a->zero_point)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: ZeroPoint must be nil for NF4 quantization scheme");
  if (a->block_axis != 0 && a->block_axis != 1)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: BlockAxis must be 0 or 1, got %d", a->block_axis);
  if (a->block_size < 1)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: BlockSize must be >= 1, got %d", a->block_size);
  if (a->activation < MX_ACT_NONE || a->activation > MX_ACT_TANH)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: unknown activation %d", a->activation);
  if (a->M < 0 || a->K < 0 || a->N < 0)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: negative size M=%lld K=%lld N=%lld",
                     (long long)a->M, (long long)a->K, (long long)a->N);
  if (a->K > (int64_t)1 << 31 || a->N > (int64_t)1 << 31)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: K and N must be < 2^31");
  int64_t outs = a->M * a->N;
  if (outs > 0 && (!a->out || (a->K > 0 && (!a->x || !a->w || !a->scale))))
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: NULL data pointer");
  d->x = a->x; d->w = a->w; d->scale = a->scale; d->zp = a->zero_point; d->bias = a->bias; d->out = a->out;
  d->M = a->M; d->K = a->K; d->N = a->N;
  d->x_dt = a->x_dtype; d->w_dt = a->w_dtype; d->s_dt = a->scale_dtype;
  d->zp_dt = a->zero_point ? a->zero_point_dtype : 0;
  d->b_dt = a->bias ? a->bias_dtype : 0;
  d->scheme = a->scheme; d->block_axis = a->block_axis; d->block_size = a->block_size; d->act = a->activation;
  return MX_OK;
}

// =============================================================================================
// Reference-order kernel.
// =============================================================================================
constexpr int kExactThreads = 256;
constexpr int kExactRows = 8;  // rows of x per thread (weights decoded once per k for all of them)

__global__ __launch_bounds__(kExactThreads) void qdense_exact_kernel(QDenseDesc d) {
  const int64_t n = (int64_t)blockIdx.x * kExactThreads + threadIdx.x;
  const int64_t m0 = (int64_t)blockIdx.y * kExactRows;
  if (n >= d.N) return;
  const int64_t N = d.N, K = d.K, B = d.block_size;
  const int rows = (int)min<int64_t>(kExactRows, d.M - m0);
  float acc[kExactRows];
  const float b0 = d.bias ? load_f(d.bias, n, d.b_dt) : 0.0f;
#pragma unroll
  for (int r = 0; r < kExactRows; ++r) acc[r] = b0;
  const int64_t nb = (N + B - 1) / B;  // reference layout: scale [K, ceil(N/B)]
  for (int64_t k = 0; k < K; ++k) {
    const int wi = decode_weight(d.w, k * N + n, d.w_dt);
    const int64_t si = d.block_axis == 1 ? k * nb + n / B : (k / B) * N + n;
    const float s = load_f(d.scale, si, d.s_dt);
    const float wf = d.scheme == MX_QUANT_NF4 ? kNF4Table[(uint32_t)wi & 15u] : (float)wi;
    if (d.zp) {
      const float z = load_f(d.zp, si, d.zp_dt);
      const float u = add_rn(mul_rn(wf, s), z);
#pragma unroll
      for (int r = 0; r < kExactRows; ++r)
        if (r < rows) acc[r] = add_rn(acc[r], mul_rn(load_f(d.x, (m0 + r) * K + k, d.x_dt), u));
    } else {
#pragma unroll
      for (int r = 0; r < kExactRows; ++r)
        if (r < rows)
          acc[r] = add_rn(acc[r], mul_rn(mul_rn(load_f(d.x, (m0 + r) * K + k, d.x_dt), wf), s));
    }
  }
#pragma unroll
  for (int r = 0; r < kExactRows; ++r)
    if (r < rows) store_f(d.out, (m0 + r) * N + n, d.x_dt, act_ref(acc[r], d.act));
}

// =============================================================================================
// Decode GEMV (M = 1, bf16 activations).
//
// Work decomposition.  A workgroup (4 waves) owns a column block of CB columns and a K slice
// of 256 rows; each wave owns 64 consecutive rows of the slice.  Lane (rho = lane/8, c = lane%8)
// reads 16 bytes (32 int4 or 16 int8 columns) of rows k and k+1 for k = kw + 16i + 2rho,
// i = 0..3: every load instruction of a wave covers 8 rows x 128 contiguous bytes, and each lane
// has 8 independent 16-byte loads in flight before it computes.
//
// Dequantisation.  v_dot2_f32_bf16 multiplies bf16 pairs, so the two rows k, k+1 of one column
// are interleaved into one dword: v_perm picks the bytes of both rows, then an and/xor turns a
// nibble u into the bf16 bit pattern 0x4300|u = 128+u (exact).  For signed int4 the xor also
// flips bit 3, so the value is 136+w.  The wave subtracts 136*sum(x) once at the end; int8
// weights are converted exactly through f32 instead (no offset).
//
// Scales.  A wave's 64 rows lie in one scale group (block_size % 64 == 0), so each lane scales
// its 32 partial sums once.  The 4 waves x 8 rho partials are summed through LDS; with more
// than one K slice the workgroup writes its column partials to scratch and the last workgroup
// to arrive for the column block adds them in slice order (deterministic), then applies bias,
// activation and the bf16 rounding.
// =============================================================================================
constexpr int kGemvThreads = 256;
constexpr int kGemvWaveRows = 64;
constexpr int kGemvSliceRows = 4 * kGemvWaveRows;

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b),
                                         c, false);
}

// Maps a workgroup index to a work item so that consecutive items (the K slices of one column
// block) land on the same XCD: workgroups are dispatched round-robin over the 8 XCDs.
__device__ __forceinline__ int xcd_swizzle(int bid, int total) {
  if ((total & 7) != 0) return bid;
  return (bid & 7) * (total >> 3) + (bid >> 3);
}

struct GemvArgs {
  const uint16_t* x;
  const uint8_t* w;
  const void* scale;
  const void* bias;
  uint16_t* out;
  float* partial;       // [S, N]
  uint32_t* counters;   // [num_cb]
  int K, N, G, S, act, b_dt;
};

template <int WDT, int SDT>
__global__ __launch_bounds__(kGemvThreads) void gemv_dot2_kernel(GemvArgs a) {
  constexpr bool kI4 = (WDT == MX_DTYPE_INT4 || WDT == MX_DTYPE_UINT4);
  constexpr int kCols = kI4 ? 32 : 16;   // columns per lane (16 bytes)
  constexpr int kCB = 8 * kCols;         // columns per workgroup
  constexpr float kOffset = WDT == MX_DTYPE_INT4 ? 136.0f : (WDT == MX_DTYPE_UINT4 ? 128.0f : 0.0f);
  constexpr uint32_t kXor = WDT == MX_DTYPE_INT4 ? 0x43084308u : 0x43004300u;
  __shared__ float red[4 * 8][kCB + 4];
  __shared__ int s_last;

  const int item = xcd_swizzle(blockIdx.x, gridDim.x);
  const int cb = item / a.S, slice = item % a.S;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rho = lane >> 3, c = lane & 7;
  const int kw = slice * kGemvSliceRows + wave * kGemvWaveRows;
  const size_t row_bytes = kI4 ? (size_t)a.N / 2 : (size_t)a.N;

  const uint8_t* wp = a.w + (size_t)(kw + 2 * rho) * row_bytes + (size_t)cb * 128 + c * 16;
  uint4 ra[4], rb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ra[i] = *(const uint4*)(wp + (size_t)(16 * i) * row_bytes);
    rb[i] = *(const uint4*)(wp + (size_t)(16 * i + 1) * row_bytes);
  }
  uint32_t xp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xp[i] = *(const uint32_t*)(a.x + kw + 16 * i + 2 * rho);

  float acc[kCols];
#pragma unroll
  for (int j = 0; j < kCols; ++j) acc[j] = 0.0f;

#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t A[4] = {ra[i].x, ra[i].y, ra[i].z, ra[i].w};
    const uint32_t Bv[4] = {rb[i].x, rb[i].y, rb[i].z, rb[i].w};
#pragma unroll
    for (int dw = 0; dw < 4; ++dw) {
      if constexpr (kI4) {
        // Bytes of rows k (A) and k+1 (B): T0 = [A.b0, A.b2, B.b0, B.b2], T1 = [A.b1, A.b3, B.b1, B.b3].
        const uint32_t t0 = __builtin_amdgcn_perm(Bv[dw], A[dw], 0x06040200u);
        const uint32_t t1 = __builtin_amdgcn_perm(Bv[dw], A[dw], 0x07050301u);
        // Nibble positions inside each 16-bit half: T0 -> columns 0,1,4,5; T1 -> 2,3,6,7.
        float* ac = acc + dw * 8;
        ac[0] = dot2_bf16(((t0 >> 0) & 0x000F000Fu) ^ kXor, xp[i], ac[0]);
        ac[1] = dot2_bf16(((t0 >> 4) & 0x000F000Fu) ^ kXor, xp[i], ac[1]);
        ac[4] = dot2_bf16(((t0 >> 8) & 0x000F000Fu) ^ kXor, xp[i], ac[4]);
        ac[5] = dot2_bf16(((t0 >> 12) & 0x000F000Fu) ^ kXor, xp[i], ac[5]);
        ac[2] = dot2_bf16(((t1 >> 0) & 0x000F000Fu) ^ kXor, xp[i], ac[2]);
        ac[3] = dot2_bf16(((t1 >> 4) & 0x000F000Fu) ^ kXor, xp[i], ac[3]);
        ac[6] = dot2_bf16(((t1 >> 8) & 0x000F000Fu) ^ kXor, xp[i], ac[6]);
        ac[7] = dot2_bf16(((t1 >> 12) & 0x000F000Fu) ^ kXor, xp[i], ac[7]);
      } else {
        float* ac = acc + dw * 4;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          float f0, f1;
          if constexpr (WDT == MX_DTYPE_INT8) {
            f0 = (float)(int8_t)(A[dw] >> (8 * p));
            f1 = (float)(int8_t)(Bv[dw] >> (8 * p));
          } else {
            f0 = (float)(uint8_t)(A[dw] >> (8 * p));
            f1 = (float)(uint8_t)(Bv[dw] >> (8 * p));
          }
          // High halves of the two f32 values are their exact bf16 encodings (|w| < 256).
          const uint32_t pair = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
          ac[p] = dot2_bf16(pair, xp[i], ac[p]);
        }
      }
    }
  }

  // Remove the magic offset, then apply the group scale of this wave's rows.
  float sx = 0.0f;
  if constexpr (kOffset != 0.0f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) sx += bf16_to_f32((uint16_t)(xp[i] & 0xFFFF)) + bf16_to_f32((uint16_t)(xp[i] >> 16));
  }
  const int g = kw / a.G;
  const int col0 = cb * kCB + c * kCols;
  if constexpr (SDT == MX_DTYPE_BFLOAT16) {
    const uint4* sp = (const uint4*)((const uint16_t*)a.scale + (size_t)g * a.N + col0);
#pragma unroll
    for (int q = 0; q < kCols / 8; ++q) {
      const uint4 v = sp[q];
      const uint32_t sv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[q * 8 + 2 * e] = (acc[q * 8 + 2 * e] - kOffset * sx) * bf16_to_f32((uint16_t)(sv[e] & 0xFFFF));
        acc[q * 8 + 2 * e + 1] = (acc[q * 8 + 2 * e + 1] - kOffset * sx) * bf16_to_f32((uint16_t)(sv[e] >> 16));
      }
    }
  } else {
    const float4* sp = (const float4*)((const float*)a.scale + (size_t)g * a.N + col0);
#pragma unroll
    for (int q = 0; q < kCols / 4; ++q) {
      const float4 v = sp[q];
      acc[q * 4 + 0] = (acc[q * 4 + 0] - kOffset * sx) * v.x;
      acc[q * 4 + 1] = (acc[q * 4 + 1] - kOffset * sx) * v.y;
      acc[q * 4 + 2] = (acc[q * 4 + 2] - kOffset * sx) * v.z;
      acc[q * 4 + 3] = (acc[q * 4 + 3] - kOffset * sx) * v.w;
    }
  }

  // Sum the 32 (wave, rho) partials of every column through LDS.
  float* myrow = &red[wave * 8 + rho][c * kCols];
#pragma unroll
  for (int j = 0; j < kCols; j += 4) *(float4*)(myrow + j) = make_float4(acc[j], acc[j + 1], acc[j + 2], acc[j + 3]);
  __syncthreads();
  const int t = threadIdx.x;
  float v = 0.0f;
  if (t < kCB) {
#pragma unroll 8
    for (int r = 0; r < 32; ++r) v += red[r][t];
  }
  const int n = cb * kCB + t;

  if (a.S == 1) {
    if (t < kCB) {
      if (a.bias) v += load_f(a.bias, n, a.b_dt);
      a.out[n] = f32_to_bf16(act_ref(v, a.act));
    }
    return;
  }

  if (t < kCB) a.partial[(size_t)slice * a.N + n] = v;
  if (!splitk_last_arriver(&a.counters[cb], (uint32_t)a.S, &s_last)) return;
  if (t < kCB) {
    float y = 0.0f;
    for (int s = 0; s < a.S; ++s) y += a.partial[(size_t)s * a.N + n];
    if (a.bias) y += load_f(a.bias, n, a.b_dt);
    a.out[n] = f32_to_bf16(act_ref(y, a.act));
  }
}

// =============================================================================================
// Kernel selection.
// =============================================================================================
enum class QPath { kEmpty, kExact, kGemvDot2, kSkinny, kGemm };

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

static QPath choose_path(const QDenseDesc& d) {
  if (d.M == 0 || d.N == 0) return QPath::kEmpty;
  if (qdense_skinny_fits(d)) return QPath::kSkinny;
  if (qdense_gemm_fits(d)) return QPath::kGemm;
  const bool i4 = d.w_dt == MX_DTYPE_INT4 || d.w_dt == MX_DTYPE_UINT4;
  const int64_t cb = i4 ? 256 : 128;
  if (d.M == 1 && d.x_dt == MX_DTYPE_BFLOAT16 && d.scheme == MX_QUANT_LINEAR && !d.zp && d.block_axis == 0 &&
      d.K > 0 && d.K % kGemvSliceRows == 0 && d.N % cb == 0 && d.block_size % kGemvWaveRows == 0 &&
      aligned(d.w, 16) && aligned(d.x, 4) && aligned(d.scale, 16))
    return QPath::kGemvDot2;
  return QPath::kExact;
}

static const char* path_name(const QDenseDesc& d, QPath p) {
  switch (p) {
    case QPath::kEmpty: return "empty";
    case QPath::kGemm:
      return d.w_dt == MX_DTYPE_INT8 ? "qdense_gemm_mfma_i8" : "qdense_gemm_mfma_u8";
    case QPath::kSkinny:
      switch (d.w_dt) {
        case MX_DTYPE_INT4: return "qdense_skinny_mfma_i4";
        case MX_DTYPE_UINT4: return "qdense_skinny_mfma_u4";
        case MX_DTYPE_INT8: return "qdense_skinny_mfma_i8";
        default: return "qdense_skinny_mfma_u8";
      }
    case QPath::kGemvDot2:
      switch (d.w_dt) {
        case MX_DTYPE_INT4: return "qdense_gemv_dot2_i4";
        case MX_DTYPE_UINT4: return "qdense_gemv_dot2_u4";
        case MX_DTYPE_INT8: return "qdense_gemv_dot2_i8";
        default: return "qdense_gemv_dot2_u8";
      }
    default: return "qdense_exact";
  }
}

int qdense_plan_name(mx_backend* b, const QDenseDesc& d, std::string* name) {
  (void)b;
  *name = path_name(d, choose_path(d));
  return MX_OK;
}

template <int WDT>
static void launch_gemv(const GemvArgs& ga, int grid, int sdt, hipStream_t st) {
  if (sdt == MX_DTYPE_BFLOAT16)
    gemv_dot2_kernel<WDT, MX_DTYPE_BFLOAT16><<<grid, kGemvThreads, 0, st>>>(ga);
  else
    gemv_dot2_kernel<WDT, MX_DTYPE_FLOAT32><<<grid, kGemvThreads, 0, st>>>(ga);
}

int qdense_run(mx_backend* b, const QDenseDesc& d) {
  MX_TRY(check_device(b));
  const QPath p = choose_path(d);
  const char* name = path_name(d, p);
  hipStream_t st = b->stream;
  switch (p) {
    case QPath::kEmpty:
      return MX_OK;
    case QPath::kSkinny:
      return qdense_skinny_run(b, d, name);
    case QPath::kGemm:
      return qdense_gemm_run(b, d, name);
    case QPath::kGemvDot2: {
      const bool i4 = d.w_dt == MX_DTYPE_INT4 || d.w_dt == MX_DTYPE_UINT4;
      const int cbw = i4 ? 256 : 128;
      const int num_cb = (int)(d.N / cbw);
      const int S = (int)(d.K / kGemvSliceRows);
      const size_t counter_bytes = 64 * 1024;
      if ((size_t)num_cb * 4 > counter_bytes)
        return set_error(MX_ERR_INVALID, "FusedQuantizedDense: N=%lld too large for the GEMV path", (long long)d.N);
      void* scratch = nullptr;
      MX_TRY(ensure_scratch(b, counter_bytes + (size_t)S * d.N * sizeof(float), &scratch));
      GemvArgs ga;
      ga.x = (const uint16_t*)d.x;
      ga.w = (const uint8_t*)d.w;
      ga.scale = d.scale;
      ga.bias = d.bias;
      ga.out = (uint16_t*)d.out;
      ga.counters = (uint32_t*)scratch;
      ga.partial = (float*)((char*)scratch + counter_bytes);
      ga.K = (int)d.K;
      ga.N = (int)d.N;
      ga.G = (int)std::min<int64_t>(d.block_size, d.K);
      ga.S = S;
      ga.act = d.act;
      ga.b_dt = d.b_dt;
      const int grid = num_cb * S;
      return launch(b, name, [&] {
        switch (d.w_dt) {
          case MX_DTYPE_INT4: launch_gemv<MX_DTYPE_INT4>(ga, grid, d.s_dt, st); break;
          case MX_DTYPE_UINT4: launch_gemv<MX_DTYPE_UINT4>(ga, grid, d.s_dt, st); break;
          case MX_DTYPE_INT8: launch_gemv<MX_DTYPE_INT8>(ga, grid, d.s_dt, st); break;
          default: launch_gemv<MX_DTYPE_UINT8>(ga, grid, d.s_dt, st); break;
        }
      });
    }
    default: {
      dim3 grid((unsigned)((d.N + kExactThreads - 1) / kExactThreads),
                (unsigned)((d.M + kExactRows - 1) / kExactRows));
      if (grid.y > 65535u) return set_error(MX_ERR_INVALID, "FusedQuantizedDense: M too large for the exact path");
      return launch(b, name, [&] { qdense_exact_kernel<<<grid, kExactThreads, 0, st>>>(d); });
    }
  }
}

}  // namespace mx

// =============================================================================================
// C ABI: direct entry points.
// =============================================================================================
extern "C" int mx_qdense(mx_backend* b, const mx_qdense_args* args) {
  mx::clear_error();
  MX_TRY(mx::check_device(b));
  mx::QDenseDesc d;
  MX_TRY(mx::qdense_validate(args, &d));
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  return mx::qdense_run(b, d);
}

extern "C" int mx_qdense_plan(mx_backend* b, const mx_qdense_args* args, char* buf, size_t buflen) {
  mx::clear_error();
  if (!b) return mx::set_error(MX_ERR_INVALID, "backend is NULL");
  mx::QDenseDesc d;
  MX_TRY(mx::qdense_validate(args, &d));
  std::string name;
  MX_TRY(mx::qdense_plan_name(b, d, &name));
  if (buf && buflen) {
    size_t n = std::min(buflen - 1, name.size());
    memcpy(buf, name.data(), n);
    buf[n] = 0;
  }
  return MX_OK;
}
