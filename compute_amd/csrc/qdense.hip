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
// Kernels (selected in this order):
//   qdense_skinny_mfma (qdense_skinny.hip) — M <= 16 bf16 rows (decode, small batches), scales
//                    blocked along K: HBM-bound streaming of the weights into MFMA operands.
//   qdense_gemm_mfma (qdense_gemm.hip) — M > 16 bf16 rows, int8/uint8/int4/uint4 weights, one
//                    scale per output column or per group of 64k rows (prefill): bf16 MFMA GEMM
//                    with on-the-fly dequantisation.
//   qdense_gemv (qdense_gemv.hip) — up to 64 rows of the reference's own layout, f32 x, zero
//                    points, NF4: HBM-bound decode GEMV.
//   qdense_refgemm_f32_mfma (qdense_refgemm.hip) — the same variants past the GEMV: f32 MFMA
//                    GEMM with each K block of weights dequantised into LDS.
//   qdense_exact   — one output column per thread, k in order, each term rounded exactly as the
//                    reference loop rounds it: bit-identical to the reference's f32 result.
//                    Used for f32 activations and every shape/layout without a fast path.

#include <algorithm>
#include <string>
#include <type_traits>

#include "device_common.h"
#include "mxrt_internal.h"

namespace mx {

// =============================================================================================
// Validation.
// =============================================================================================
static bool is_f32_or_bf16(int dt) { return dt == MX_DTYPE_FLOAT32 || dt == MX_DTYPE_BFLOAT16; }

// FusedQuantizedDenseGGML's checks (quantizeddense.go:181-248) on the direct entry point's args.
static int ggml_validate(const mx_qdense_args* a, QDenseDesc* d) {
  const char* op = "FusedQuantizedDense(GGML)";
  int vpb, bpb;
  switch (a->ggml_type) {
    case MX_GGML_Q4_0: case MX_GGML_Q8_0: case MX_GGML_IQ4_NL: case MX_GGML_Q4_K: case MX_GGML_Q6_K: break;
    default: return set_error(MX_ERR_NOT_IMPLEMENTED, "%s: GGML type %d not supported in fused path", op, a->ggml_type);
  }
  MX_TRY(ggml_block_geometry(a->ggml_type, &vpb, &bpb));
  if (a->x_dtype != MX_DTYPE_FLOAT32)
    return set_error(MX_ERR_INVALID, "%s: x must be float32, got %s", op, dtype_name(a->x_dtype));
  if (a->zero_point) return set_error(MX_ERR_INVALID, "%s: ZeroPoint must be nil for GGML scheme", op);
  if (a->bias && a->bias_dtype != MX_DTYPE_FLOAT32)
    return set_error(MX_ERR_INVALID, "%s: bias must be float32, got %s", op, dtype_name(a->bias_dtype));
  if (a->activation < MX_ACT_NONE || a->activation > MX_ACT_TANH)
    return set_error(MX_ERR_INVALID, "%s: unknown activation %d", op, a->activation);
  if (a->M < 0 || a->K < 0 || a->N < 0 || a->K % vpb != 0)
    return set_error(MX_ERR_INVALID, "%s: K=%lld must be a non-negative multiple of %d (M=%lld, N=%lld)", op,
                     (long long)a->K, vpb, (long long)a->M, (long long)a->N);
  if (a->K >= (int64_t)1 << 31 || a->N >= (int64_t)1 << 31) return set_error(MX_ERR_INVALID, "%s: K and N must be < 2^31", op);
  if (a->M * a->N > 0 && (!a->out || (a->K > 0 && (!a->x || !a->w))))
    return set_error(MX_ERR_INVALID, "%s: NULL data pointer", op);
  *d = QDenseDesc{};
  d->x = a->x; d->w = a->w; d->bias = a->bias; d->out = a->out;
  d->M = a->M; d->K = a->K; d->N = a->N;
  d->x_dt = MX_DTYPE_FLOAT32; d->w_dt = MX_DTYPE_UINT8; d->b_dt = a->bias ? MX_DTYPE_FLOAT32 : 0;
  d->scheme = MX_QUANT_GGML; d->act = a->activation;
  d->ggml_type = a->ggml_type;
  d->bpr = a->K / vpb * bpb;
  return MX_OK;
}

int qdense_validate(const mx_qdense_args* a, QDenseDesc* d) {
  if (!a) return set_error(MX_ERR_INVALID, "FusedQuantizedDense: args is NULL");
  if (a->scheme == MX_QUANT_GGML) return ggml_validate(a, d);
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
  if (a->K >= (int64_t)1 << 31 || a->N >= (int64_t)1 << 31)
    return set_error(MX_ERR_INVALID, "FusedQuantizedDense: K and N must be < 2^31");
  // Element alignment (what a Go slice of the dtype always has): f32 on 4 bytes, bf16 on 2.
  auto misaligned = [](const void* p, int dt) {
    return p && ((uintptr_t)p % (uintptr_t)(dt == MX_DTYPE_FLOAT32 ? 4 : 2)) != 0;
  };
  if (misaligned(a->x, a->x_dtype) || misaligned(a->scale, a->scale_dtype) ||
      (a->zero_point && misaligned(a->zero_point, a->zero_point_dtype)) ||
      (a->bias && misaligned(a->bias, a->bias_dtype)) || misaligned(a->out, a->x_dtype))
    return set_error(MX_ERR_INVALID,
                     "FusedQuantizedDense: float32 data must be 4-byte aligned and bfloat16 data 2-byte aligned");
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
// Reference-order kernel: every output is summed exactly as the reference loop sums it (bias
// first, then k in increasing order, each product and sum rounded on its own), so the result is
// bit-identical.  That order is a chain per output; the kernel keeps the chain fed instead of
// waiting on memory at every k:
//   - a thread computes R rows of one column (R = 8 amortises the weight decoding when the grid
//     has waves to spare, R = 1 spreads a small problem over more waves);
//   - the workgroup's rows of x are staged in LDS, kExactKC values per row at a time;
//   - the weights and scales of a batch of consecutive k (16 or 64) are requested as raw bytes/bits one batch
//     ahead (two register slots), and decoded only when they are used.
// =============================================================================================
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kExactThreads = 256;
constexpr int kExactKC = 512;  // x values per row staged in LDS at a time
constexpr int kExactU = 16;    // k per batch of weight / scale requests (see U)

// Branch-free operand access for the reference-order loop (the dtypes are run-time values, and a
// branch per dtype per k would make the unrolled loop too large for the instruction cache):
//   - weight element i lives in byte i / 2 (4-bit kinds: nibble i % 2) or byte i, and is one
//     signed or unsigned bit-field extract of that byte;
//   - a bf16 or f32 element (scales, zero points) is read as the aligned 32-bit word holding it
//     and shifted into f32 position (bf16 widened exactly).
// Element indices advance by a constant per k: no multiplication or division per k.
// The word is the aligned one that holds the element's absolute address (bf16 arrays need only be
// 2-byte aligned), so the load never leaves the element's own 4 bytes.
__device__ __forceinline__ uint32_t word_of(const void* p, uint64_t i, int sh) {
  return *(const uint32_t*)(((uintptr_t)p + (i << sh)) & ~(uintptr_t)3);
}
// The f32 value of element i from its word: f32 (sh 2) as is, bf16 (sh 1) moved to the high half
// when it sits in the word's low half.  podd: bit 1 of the array's address (an array that starts
// 2 bytes into a word has its even elements in high halves).
__device__ __forceinline__ uint32_t word_shift(uint64_t i, int sh, uint32_t podd) {
  return sh == 2 || ((i ^ podd) & 1) ? 0u : 16u;
}
__device__ __forceinline__ float word_value(uint32_t w, uint32_t shift, uint32_t mask) {
  return __uint_as_float((w << shift) & mask);
}

// R: rows per thread.  ZP: zero points.  SK: the scale varies along K (groups or the reference
// layout); else one scale per column, loaded once.
template <int R, bool ZP, bool SK>
__global__ __launch_bounds__(kExactThreads) void qdense_exact_kernel(QDenseDesc d) {
  // k per batch of requests: 64 when a thread has one row and one scale per column (few waves
  // per SIMD, latency hidden only by the batch), else 16 (registers).
  constexpr int U = R == 1 && !SK ? 64 : kExactU;
  static_assert(kExactKC % (2 * U) == 0, "batches tile a chunk");
  __shared__ __attribute__((aligned(16))) float xs[R][kExactKC];
  __shared__ float nf4[16];
  const int64_t N = d.N, K = d.K, B = d.block_size;
  const int64_t n = (int64_t)blockIdx.x * kExactThreads + threadIdx.x;
  const int64_t m0 = (int64_t)blockIdx.y * R;
  const bool active = n < N;
  const int64_t nn = active ? n : 0;  // lanes past N read column 0; their results are not stored
  const int rows = (int)min<int64_t>(R, d.M - m0);
  const bool packed = d.w_dt == MX_DTYPE_INT4 || d.w_dt == MX_DTYPE_UINT4;
  const bool sgn = d.w_dt == MX_DTYPE_INT4 || d.w_dt == MX_DTYPE_INT8;
  const uint32_t wbits = packed ? 4u : 8u, wsh = packed ? 1u : 0u;
  const int s_sh = d.s_dt == MX_DTYPE_BFLOAT16 ? 1 : 2, z_sh = d.zp_dt == MX_DTYPE_BFLOAT16 ? 1 : 2;
  const uint32_t s_mask = s_sh == 2 ? ~0u : 0xFFFF0000u, z_mask = z_sh == 2 ? ~0u : 0xFFFF0000u;
  const uint32_t s_odd = (uint32_t)((uintptr_t)d.scale >> 1) & 1u, z_odd = (uint32_t)((uintptr_t)d.zp >> 1) & 1u;
  const bool nf = d.scheme == MX_QUANT_NF4;
  if (threadIdx.x < 16) nf4[threadIdx.x] = kNF4Table[threadIdx.x];
  // Scale (and zero point) of row k: block_axis 1 (reference layout, [K, ceil(N/B)]) at
  // k * nb + n / B, stepping by nb; block_axis 0 ([ceil(K/B), N]) at (k / B) * N + n, stepping by
  // N at each group's end.
  const bool ax1 = d.block_axis == 1;
  const int64_t nb = (N + B - 1) / B;
  const int64_t scol = ax1 ? (int64_t)((uint32_t)nn / (uint32_t)B) : nn;
  float s_col = 0.0f, z_col = 0.0f;  // one scale per column (SK false)
  if constexpr (!SK) {
    s_col = word_value(word_of(d.scale, (uint64_t)scol, s_sh), word_shift((uint64_t)scol, s_sh, s_odd), s_mask);
    if constexpr (ZP)
      z_col = word_value(word_of(d.zp, (uint64_t)scol, z_sh), word_shift((uint64_t)scol, z_sh, z_odd), z_mask);
  }
  float acc[R];
  const float b0 = d.bias ? load_f(d.bias, nn, d.b_dt) : 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = b0;

  // Operands of U consecutive k as raw bytes / words, decoded when used.
  struct Batch {
    uint32_t w[U], s[U], z[U], ssh[U], zsh[U];
    uint32_t off0, off1;  // bit offset of the weight in its byte at even / odd j
  };
  // Running element indices of the next k to request: weight k * N + n, scale / zero point.
  uint64_t wi = 0, si = 0;
  uint32_t gr = 0;  // block_axis 0: place of k in its group
  auto start = [&](int k) {
    wi = (uint64_t)k * (uint64_t)N + (uint64_t)nn;
    if (ax1) {
      si = (uint64_t)k * (uint64_t)nb + (uint64_t)scol;
    } else {
      const uint32_t g = (uint32_t)k / (uint32_t)B;
      gr = (uint32_t)k - g * (uint32_t)B;
      si = (uint64_t)g * (uint64_t)N + (uint64_t)scol;
    }
  };
  const uint32_t nodd = (uint32_t)N & 1u;
  auto step_scale = [&]() __attribute__((always_inline)) {
    if (ax1) {
      si += (uint64_t)nb;
    } else if (++gr == (uint32_t)B) {
      gr = 0;
      si += (uint64_t)N;
    }
  };
  // Requests k0 .. k0 + U - 1 (FULL: all below kend; else those at or past kend repeat
  // kend - 1 and are not used).
  auto issue = [&](Batch& bt, int k0, int kend, auto fullc) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(fullc)::value;
    // The nibble of element wi + j * N: that of wi, flipped at odd j when N is odd.
    const uint32_t h0 = packed ? (uint32_t)wi & 1u : 0u;
    bt.off0 = 4u * h0;
    bt.off1 = 4u * (h0 ^ (packed ? nodd : 0u));
#pragma unroll
    for (int j = 0; j < U; ++j) {
      bt.w[j] = ((const uint8_t*)d.w)[wi >> wsh];
      if constexpr (SK) {
        bt.s[j] = word_of(d.scale, si, s_sh);
        bt.ssh[j] = word_shift(si, s_sh, s_odd);
        if constexpr (ZP) {
          bt.z[j] = word_of(d.zp, si, z_sh);
          bt.zsh[j] = word_shift(si, z_sh, z_odd);
        }
      }
      if (FULL || k0 + j + 1 < kend) {
        wi += (uint64_t)N;
        if constexpr (SK) step_scale();
      }
    }
  };
  auto compute = [&](const Batch& bt, int k0, int kend, int kc, auto fullc) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(fullc)::value;
    // Weight values of the batch (NF4: through the table), then the terms in k order.
    float wf[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const uint32_t off = (j & 1) ? bt.off1 : bt.off0;
      const int wv = sgn ? __builtin_amdgcn_sbfe((int)bt.w[j], off, wbits) : (int)__builtin_amdgcn_ubfe(bt.w[j], off, wbits);
      wf[j] = (float)wv;
    }
    if (nf) {
#pragma unroll
      for (int j = 0; j < U; ++j) wf[j] = nf4[(uint32_t)(int)wf[j] & 15u];
    }
#pragma unroll
    for (int j4 = 0; j4 < U; j4 += 4) {
      float xv[R][4];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const f32x4_t v = *(const f32x4_t*)&xs[r][k0 + j4 - kc];
#pragma unroll
        for (int q = 0; q < 4; ++q) xv[r][q] = v[q];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j = j4 + q;
        if (FULL || k0 + j < kend) {
          float s, z = 0.0f;
          if constexpr (SK) {
            s = word_value(bt.s[j], bt.ssh[j], s_mask);
            if constexpr (ZP) z = word_value(bt.z[j], bt.zsh[j], z_mask);
          } else {
            s = s_col;
            z = z_col;
          }
          if constexpr (ZP) {
            const float u = add_rn(mul_rn(wf[j], s), z);
#pragma unroll
            for (int r = 0; r < R; ++r)
              if (r < rows) acc[r] = add_rn(acc[r], mul_rn(xv[r][q], u));
          } else {
#pragma unroll
            for (int r = 0; r < R; ++r)
              if (r < rows) acc[r] = add_rn(acc[r], mul_rn(mul_rn(xv[r][q], wf[j]), s));
          }
        }
      }
    }
  };
  using Full = std::integral_constant<bool, true>;
  using Part = std::integral_constant<bool, false>;
  auto issue_any = [&](Batch& bt, int k0, int kend) __attribute__((always_inline)) {
    if (k0 + U <= kend)
      issue(bt, k0, kend, Full{});
    else
      issue(bt, k0, kend, Part{});
  };
  auto compute_any = [&](const Batch& bt, int k0, int kend, int kc) __attribute__((always_inline)) {
    if (k0 + U <= kend)
      compute(bt, k0, kend, kc, Full{});
    else
      compute(bt, k0, kend, kc, Part{});
  };

  const int Ki = (int)K;  // K < 2^31 (validated)
  for (int kc = 0; kc < Ki; kc += kExactKC) {
    const int kend = min(Ki, kc + kExactKC);
    const int kn = kend - kc;
    __syncthreads();  // the previous chunk's x has been used (and the NF4 table written)
    for (int i = threadIdx.x; i < R * kExactKC; i += kExactThreads) {
      const int r = i / kExactKC, j = i - r * kExactKC;
      xs[r][j] = r < rows && j < kn ? load_f(d.x, (m0 + r) * K + kc + j, d.x_dt) : 0.0f;
    }
    __syncthreads();
    // Two batches of requests in flight: batch b + 1 is requested before batch b is computed.
    start(kc);
    Batch A, Bt;
    issue_any(A, kc, kend);
    for (int k0 = kc; k0 < kend; k0 += 2 * U) {
      const bool more = k0 + U < kend;
      if (more) issue_any(Bt, k0 + U, kend);
      compute_any(A, k0, kend, kc);
      if (k0 + 2 * U < kend) issue_any(A, k0 + 2 * U, kend);
      if (more) compute_any(Bt, k0 + U, kend, kc);
    }
  }
  if (!active) return;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (r < rows) store_f(d.out, (m0 + r) * N + n, d.x_dt, act_ref(acc[r], d.act));
}

// Rows per thread of the reference-order kernel: 8 when the grid has two waves per SIMD of a
// 256-CU part even so, else 1.
static int exact_rows(const QDenseDesc& d) {
  const int64_t col_blocks = (d.N + kExactThreads - 1) / kExactThreads;
  return d.M * col_blocks * (kExactThreads / 64) > 2048 ? 8 : 1;
}

// =============================================================================================
// Reference layout and variants at prefill size (scale [K, ceil(N/B)] with BlockAxis = 1, f32 x,
// zero points, NF4): the fused dequantise-and-contract kernel of qdense_refgemm.hip (f32 matrix
// cores, the weights dequantised per K block into LDS).  Problems of at most 2^24 multiply-adds
// keep the exact kernel (the reference's own BenchmarkQuantizedDense shapes, up to
// 32 x 512 x 1024, stay bit-identical to it).
// =============================================================================================
constexpr int64_t kRefGemmMinMKN = (int64_t)1 << 24;

static bool qdense_refgemm_plan(const QDenseDesc& d) {
  return d.M > 4 && d.M * d.K * d.N > kRefGemmMinMKN && qdense_refgemm_fits(d);
}

// =============================================================================================
// Kernel selection.
// =============================================================================================
enum class QPath { kEmpty, kExact, kSkinny, kSkinnyRows, kGemv, kGemm, kRefGemm };

// Past 16 rows of bf16 x: the skinny kernel once per group of 16 rows (its row limit).  Each
// launch streams the weights once at decode rate (13-17 us per 16 rows at [4096] x 11008-14336
// columns), while the GEMM's 256-row tiles are mostly padding at these M and its 128- or
// 64-column tiles leave most CUs without work: one GEMM launch costs about 51 us there with
// per-channel scales and 71-102 us with scale groups, so up to 3 (per-channel) or 4 (grouped)
// skinny launches cost less.
constexpr int64_t kSkinnyRowsPerLaunch = 16;

static bool skinny_rows_fit(const QDenseDesc& d) {
  const int64_t launches = d.block_size < d.K ? 4 : 3;
  if (d.M <= kSkinnyRowsPerLaunch || d.M > launches * kSkinnyRowsPerLaunch) return false;
  QDenseDesc g = d;
  g.M = kSkinnyRowsPerLaunch;
  return qdense_skinny_fits(g);
}

// Past the GEMV's 64 rows, for what neither the GEMM nor the fused reference-layout kernel takes
// (rows that start mid-word: N not a multiple of the 16 columns those kernels load): the GEMV once
// per group of four rows, which reads the weights again per group.  From 2^24 weights that still
// beats the exact kernel, whose sequential multiply-adds run at about 3 TMAC/s: Int4 f32 x
// [4096] x 32001 with [K, 251] scales takes 5.7 ms (128 rows) and 22.9 ms (512 rows) in the exact
// kernel and about 11 us per row in the GEMV.
constexpr int64_t kGemvManyRowsMinWeights = (int64_t)1 << 24;

static bool gemv_many_rows_plan(const QDenseDesc& d) {
  if (d.K * d.N < kGemvManyRowsMinWeights) return false;
  QDenseDesc g = d;
  g.M = 1;  // the row count is the only limit qdense_gemv_fits applies past one row
  return qdense_gemv_fits(g);
}

static GgmlDesc ggml_desc(const QDenseDesc& d) {
  GgmlDesc g;
  g.x = (const float*)d.x;
  g.w = (const uint8_t*)d.w;
  g.bias = (const float*)d.bias;
  g.out = (float*)d.out;
  g.M = d.M;
  g.K = d.K;
  g.N = d.N;
  g.bpr = d.bpr;
  g.type = d.ggml_type;
  g.act = d.act;
  return g;
}

static QPath choose_path(const mx_backend* b, const QDenseDesc& d) {
  if (d.M == 0 || d.N == 0) return QPath::kEmpty;
  if (d.scheme == MX_QUANT_GGML || b->exact_qdense) return QPath::kExact;
  if (qdense_skinny_fits(d)) return QPath::kSkinny;
  if (!b->gemv_over_gemm && skinny_rows_fit(d)) return QPath::kSkinnyRows;
  // Past the skinny kernel's 16 rows the GEMM reads every weight once, while the GEMV reads the
  // whole weight matrix again for every 4 rows: the GEMV takes only what the GEMM does not fit.
  if (!b->gemv_over_gemm && qdense_gemm_fits(d)) return QPath::kGemm;
  if (qdense_gemv_fits(d)) return QPath::kGemv;
  if (qdense_gemm_fits(d)) return QPath::kGemm;
  // The reference layout, f32 x, zero points and NF4 at prefill size: the fused kernel.
  if (qdense_refgemm_plan(d)) return QPath::kRefGemm;
  if (gemv_many_rows_plan(d)) return QPath::kGemv;
  return QPath::kExact;
}

static const char* path_name(const QDenseDesc& d, QPath p) {
  switch (p) {
    case QPath::kEmpty: return "empty";
    case QPath::kRefGemm: return "qdense_refgemm_f32_mfma";
    case QPath::kGemm:
      switch (d.w_dt) {
        case MX_DTYPE_INT8: return d.block_size < d.K ? "qdense_gemm_mfma_i8_grouped" : "qdense_gemm_mfma_i8";
        case MX_DTYPE_UINT8: return d.block_size < d.K ? "qdense_gemm_mfma_u8_grouped" : "qdense_gemm_mfma_u8";
        case MX_DTYPE_INT4: return d.block_size < d.K ? "qdense_gemm_mfma_i4_grouped" : "qdense_gemm_mfma_i4";
        default: return d.block_size < d.K ? "qdense_gemm_mfma_u4_grouped" : "qdense_gemm_mfma_u4";
      }
    case QPath::kSkinny:
      switch (d.w_dt) {
        case MX_DTYPE_INT4: return "qdense_skinny_mfma_i4";
        case MX_DTYPE_UINT4: return "qdense_skinny_mfma_u4";
        case MX_DTYPE_INT8: return "qdense_skinny_mfma_i8";
        default: return "qdense_skinny_mfma_u8";
      }
    case QPath::kSkinnyRows:
      switch (d.w_dt) {
        case MX_DTYPE_INT4: return "qdense_skinny_rows16_i4";
        case MX_DTYPE_UINT4: return "qdense_skinny_rows16_u4";
        case MX_DTYPE_INT8: return "qdense_skinny_rows16_i8";
        default: return "qdense_skinny_rows16_u8";
      }
    case QPath::kGemv:
      if (d.scheme == MX_QUANT_NF4) return dtype_is_packed(d.w_dt) ? "qdense_gemv_nf4_4bit" : "qdense_gemv_nf4_8bit";
      switch (d.w_dt) {
        case MX_DTYPE_INT4: return d.zp ? "qdense_gemv_i4_zp" : "qdense_gemv_i4";
        case MX_DTYPE_UINT4: return d.zp ? "qdense_gemv_u4_zp" : "qdense_gemv_u4";
        case MX_DTYPE_INT8: return d.zp ? "qdense_gemv_i8_zp" : "qdense_gemv_i8";
        default: return d.zp ? "qdense_gemv_u8_zp" : "qdense_gemv_u8";
      }
    default: return "qdense_exact";
  }
}

int qdense_plan_name(mx_backend* b, const QDenseDesc& d, std::string* name) {
  if (d.scheme == MX_QUANT_GGML) {
    *name = ggml_plan_name(b, ggml_desc(d));
    return MX_OK;
  }
  const QPath p = choose_path(b, d);
  *name = path_name(d, p);
  if (d.pair) *name += p == QPath::kSkinny || p == QPath::kSkinnyRows ? "_pair" : "+" + *name + "+mul";
  return MX_OK;
}

int qdense_run(mx_backend* b, const QDenseDesc& d) {
  MX_TRY(check_device(b));
  const QPath p = choose_path(b, d);
  if (d.pair && p != QPath::kSkinny && p != QPath::kSkinnyRows && p != QPath::kEmpty) {
    // Only the skinny kernel computes a pair in one launch: elsewhere the second product goes to
    // a temporary and the first applies the product in its epilogue (the same arithmetic).
    const size_t bytes = (size_t)d.M * d.N * (d.x_dt == MX_DTYPE_BFLOAT16 ? 2 : 4);
    void* tmp = nullptr;
    MX_TRY(dev_alloc(b, bytes, &tmp));
    QDenseDesc d2 = d;
    d2.pair = false;
    d2.w = d.w2;
    d2.scale = d.scale2;
    d2.bias = d.bias2;
    d2.b_dt = d.b2_dt;
    d2.act = d.act2;
    d2.out = tmp;
    d2.res = nullptr;
    d2.res_op = 0;
    QDenseDesc d1 = d;
    d1.pair = false;
    d1.res = tmp;
    d1.res_dt = d.x_dt;
    d1.res_op = MX_OP_MUL;
    int rc = qdense_run(b, d2);
    if (rc == MX_OK) rc = qdense_run(b, d1);
    dev_free(b, tmp);  // stream-ordered pool: later users run after these kernels
    return rc;
  }
  if (d.res_op != 0 && p != QPath::kSkinny && p != QPath::kSkinnyRows && p != QPath::kEmpty) {
    // Only the skinny kernel applies a folded elementwise op in its epilogue: elsewhere the dense
    // result goes to a temporary and the op runs as its own kernel (the same arithmetic).
    const int64_t dims[2] = {d.M, d.N};
    const size_t bytes = (size_t)d.M * d.N * (d.x_dt == MX_DTYPE_BFLOAT16 ? 2 : 4);
    void* tmp = nullptr;
    MX_TRY(dev_alloc(b, bytes, &tmp));
    QDenseDesc d2 = d;
    d2.out = tmp;
    d2.res = nullptr;
    d2.res_op = 0;
    int rc = qdense_run(b, d2);
    if (rc == MX_OK) rc = ew_binary(b, d.res_op, tmp, dims, d.res, dims, d.out, dims, 2, d.x_dt);
    dev_free(b, tmp);  // stream-ordered pool: later users run after these kernels
    return rc;
  }
  if (d.scheme == MX_QUANT_GGML) return ggml_dense_run(b, ggml_desc(d));
  const char* name = path_name(d, p);
  hipStream_t st = b->stream;
  switch (p) {
    case QPath::kEmpty:
      return MX_OK;
    case QPath::kSkinny:
      return qdense_skinny_run(b, d, name);
    case QPath::kSkinnyRows: {
      // bf16 x and output; the elementwise operand has the output's shape.
      const int64_t re = d.res ? dtype_bits(d.res_dt) / 8 : 0;
      for (int64_t m0 = 0; m0 < d.M; m0 += kSkinnyRowsPerLaunch) {
        QDenseDesc g = d;
        g.M = std::min<int64_t>(kSkinnyRowsPerLaunch, d.M - m0);
        g.x = (const char*)d.x + m0 * d.K * 2;
        g.out = (char*)d.out + m0 * d.N * 2;
        if (d.res) g.res = (const char*)d.res + m0 * d.N * re;
        MX_TRY(qdense_skinny_run(b, g, name));
      }
      return MX_OK;
    }
    case QPath::kGemv:
      return qdense_gemv_run(b, d, name);
    case QPath::kGemm:
      return qdense_gemm_run(b, d, name);
    case QPath::kRefGemm:
      return qdense_refgemm_run(b, d, name);
    default: {
      const int R = exact_rows(d);
      dim3 grid((unsigned)((d.N + kExactThreads - 1) / kExactThreads), (unsigned)((d.M + R - 1) / R));
      if (grid.y > 65535u) return set_error(MX_ERR_INVALID, "FusedQuantizedDense: M too large for the exact path");
      // The scale varies along K unless there is one per column (block_axis 0, one group).
      const bool sk = d.block_axis == 1 || d.block_size < d.K;
      return launch(b, name, [&] {
        auto go = [&](auto kern) { dispatch(kern, grid, kExactThreads, 0, st, d); };
        if (R == 8) {
          if (d.zp)
            sk ? go(qdense_exact_kernel<8, true, true>) : go(qdense_exact_kernel<8, true, false>);
          else
            sk ? go(qdense_exact_kernel<8, false, true>) : go(qdense_exact_kernel<8, false, false>);
        } else {
          if (d.zp)
            sk ? go(qdense_exact_kernel<1, true, true>) : go(qdense_exact_kernel<1, true, false>);
          else
            sk ? go(qdense_exact_kernel<1, false, true>) : go(qdense_exact_kernel<1, false, false>);
        }
      });
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
