// Normalized DotGeneral on gfx950: out[b, m, n] = sum_k lhs[b, m, k] * rhs[b, k, n]
// (rhs[b, n, k] when transposed).  This is the kernel the reference's dot.DotGeneral lowering
// targets (internal/gobackend/dot/dot.go:165-285: [B,M,K] x [B,K,N] "NonTransposed" or
// [B,N,K] "Transposed" layouts, half-precision inputs accumulating into f32).
//
// The tiled kernel stages 64x64 output tiles through LDS, 16-deep in K, each thread owning a
// 4x4 register block; it serves f32 and f64 (accumulating in the input type) and bf16/f16
// (accumulating in f32).

#include "device_common.h"
#include "mxrt_internal.h"

namespace mx {

constexpr int kDotTile = 64;
constexpr int kDotKStep = 16;

template <typename TI, typename TA>
__device__ __forceinline__ TA load_acc(const TI* p, int64_t i, int dt) {
  if constexpr (sizeof(TI) == 2) {
    const uint16_t h = ((const uint16_t*)p)[i];
    return (TA)(dt == MX_DTYPE_BFLOAT16 ? bf16_to_f32(h) : f16_to_f32(h));
  } else {
    return (TA)p[i];
  }
}

template <typename TI, typename TA>
__global__ __launch_bounds__(256) void dot_tiled_kernel(const TI* __restrict__ lhs, const TI* __restrict__ rhs,
                                                        TA* __restrict__ out, int64_t M, int64_t K, int64_t N,
                                                        bool rhs_t, int in_dt) {
  __shared__ TA As[kDotKStep][kDotTile + 1];
  __shared__ TA Bs[kDotKStep][kDotTile + 1];
  const int64_t b = blockIdx.z;
  const int64_t m0 = (int64_t)blockIdx.y * kDotTile, n0 = (int64_t)blockIdx.x * kDotTile;
  const TI* L = lhs + b * M * K;
  const TI* R = rhs + b * K * N;
  const int tid = threadIdx.x;
  const int ty = tid / 16, tx = tid % 16;
  TA acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (TA)0;
  for (int64_t k0 = 0; k0 < K; k0 += kDotKStep) {
    // 64x16 tiles = 1024 elements, 4 per thread.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = tid + e * 256;
      {  // lhs: As[kk][mm] = L[m0+mm, k0+kk]
        const int kk = idx % kDotKStep, mm = idx / kDotKStep;
        const int64_t m = m0 + mm, k = k0 + kk;
        As[kk][mm] = (m < M && k < K) ? load_acc<TI, TA>(L, m * K + k, in_dt) : (TA)0;
      }
      if (!rhs_t) {  // Bs[kk][nn] = R[k0+kk, n0+nn]
        const int nn = idx % kDotTile, kk = idx / kDotTile;
        const int64_t n = n0 + nn, k = k0 + kk;
        Bs[kk][nn] = (n < N && k < K) ? load_acc<TI, TA>(R, k * N + n, in_dt) : (TA)0;
      } else {  // Bs[kk][nn] = R[n0+nn, k0+kk]
        const int kk = idx % kDotKStep, nn = idx / kDotKStep;
        const int64_t n = n0 + nn, k = k0 + kk;
        Bs[kk][nn] = (n < N && k < K) ? load_acc<TI, TA>(R, n * K + k, in_dt) : (TA)0;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kDotKStep; ++kk) {
      TA a[4], bb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bb[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * bb[j];
    }
    __syncthreads();
  }
  TA* O = out + b * M * N;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + ty * 4 + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n < N) O[m * N + n] = acc[i][j];
    }
  }
}

int dot_run(mx_backend* b, const DotDesc& d) {
  MX_TRY(check_device(b));
  if (d.B == 0 || d.M == 0 || d.N == 0) return MX_OK;
  if (d.K == 0) {
    const size_t bytes = (size_t)d.B * d.M * d.N * (dtype_bits(d.out_dt) / 8);
    MX_CHECK_HIP(hipMemsetAsync(d.out, 0, bytes, b->stream));
    return MX_OK;
  }
  if (dot_mfma_fits(d))
    return dot_mfma_run(b, d, d.in_dt == MX_DTYPE_BFLOAT16 ? "dot_mfma_bf16" : "dot_mfma_f16");
  if (dtype_is_half(d.in_dt) && d.out_dt != MX_DTYPE_FLOAT32) {
    // Half output folded in by the graph compiler, on a path that sums into f32 memory: the f32
    // result goes to a temporary, then ConvertDType's own kernel rounds it (the same arithmetic).
    void* tmp = nullptr;
    const int64_t n = d.B * d.M * d.N;
    MX_TRY(dev_alloc(b, (size_t)n * sizeof(float), &tmp));
    DotDesc d2 = d;
    d2.out = tmp;
    d2.out_dt = MX_DTYPE_FLOAT32;
    int rc = dot_run(b, d2);
    if (rc == MX_OK) rc = ew_convert(b, tmp, MX_DTYPE_FLOAT32, d.out, d.out_dt, n);
    dev_free(b, tmp);  // stream-ordered pool: later users run after these kernels
    return rc;
  }
  if (d.B > 65535) return set_error(MX_ERR_INVALID, "DotGeneral: batch size %lld too large", (long long)d.B);
  dim3 grid((unsigned)((d.N + kDotTile - 1) / kDotTile), (unsigned)((d.M + kDotTile - 1) / kDotTile), (unsigned)d.B);
  if (grid.y > 65535u) return set_error(MX_ERR_INVALID, "DotGeneral: M too large");
  hipStream_t st = b->stream;
  switch (d.in_dt) {
    case MX_DTYPE_FLOAT32:
      return launch(b, "dot_tiled_f32", [&] {
        dispatch(dot_tiled_kernel<float, float>, grid, 256, 0, st, (const float*)d.lhs, (const float*)d.rhs, (float*)d.out, d.M,
                                                              d.K, d.N, d.rhs_transposed, d.in_dt);
      });
    case MX_DTYPE_FLOAT64:
      return launch(b, "dot_tiled_f64", [&] {
        dispatch(dot_tiled_kernel<double, double>, grid, 256, 0, st, (const double*)d.lhs, (const double*)d.rhs,
                                                                (double*)d.out, d.M, d.K, d.N, d.rhs_transposed, d.in_dt);
      });
    case MX_DTYPE_BFLOAT16:
    case MX_DTYPE_FLOAT16:
      return launch(b, d.in_dt == MX_DTYPE_BFLOAT16 ? "dot_tiled_bf16" : "dot_tiled_f16", [&] {
        dispatch(dot_tiled_kernel<uint16_t, float>, grid, 256, 0, st, (const uint16_t*)d.lhs, (const uint16_t*)d.rhs,
                                                                 (float*)d.out, d.M, d.K, d.N, d.rhs_transposed, d.in_dt);
      });
    default:
      return set_error(MX_ERR_NOT_IMPLEMENTED, "DotGeneral: dtype %s not implemented", dtype_name(d.in_dt));
  }
}

}  // namespace mx
