// Elementwise, reduction and data-movement kernels used by graphs around the hot path (the
// quantized MLP block: RMSNorm, SiLU(gate)*up, residual add) and by DotGeneral lowering.
//
// Numeric semantics follow the reference's Go executors:
//   - unary ops evaluate in f64 and round to the storage type; half types round f64 -> f32 ->
//     half (internal/gobackend/ops/unaryops.go, e.g. :646-669 Logistic, :812-822 Rsqrt);
//   - binary ops on bf16/f16 compute in f32 and round once (gen_exec_binary.go:119-140);
//   - ReduceSum on bf16/f16 accumulates in f32 and rounds at the end (reduce.go:416-437);
//   - ConvertDType float -> bf16 uses round-to-nearest-even (bfloat16.go:30-39).

#include <algorithm>
#include <type_traits>

#include "device_common.h"
#include "mxrt_internal.h"

namespace mx {

constexpr int kEwThreads = 256;

static inline unsigned ew_blocks(int64_t n) {
  int64_t b = (n + kEwThreads - 1) / kEwThreads;
  return (unsigned)(b > 65535 * 8 ? 65535 * 8 : (b < 1 ? 1 : b));
}

// ---------------------------------------------------------------------------------------------
// Generic element access.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ double load_as_double(const void* p, int64_t i, int dt) {
  switch (dt) {
    case MX_DTYPE_FLOAT32: return ((const float*)p)[i];
    case MX_DTYPE_FLOAT64: return ((const double*)p)[i];
    case MX_DTYPE_BFLOAT16: return bf16_to_f32(((const uint16_t*)p)[i]);
    case MX_DTYPE_FLOAT16: return f16_to_f32(((const uint16_t*)p)[i]);
    case MX_DTYPE_INT8: return ((const int8_t*)p)[i];
    case MX_DTYPE_INT16: return ((const int16_t*)p)[i];
    case MX_DTYPE_INT32: return ((const int32_t*)p)[i];
    case MX_DTYPE_INT64: return (double)((const int64_t*)p)[i];
    case MX_DTYPE_UINT8: case MX_DTYPE_BOOL: return ((const uint8_t*)p)[i];
    case MX_DTYPE_UINT16: return ((const uint16_t*)p)[i];
    case MX_DTYPE_UINT32: return ((const uint32_t*)p)[i];
    case MX_DTYPE_UINT64: return (double)((const uint64_t*)p)[i];
    case MX_DTYPE_INT4: case MX_DTYPE_UINT4: return decode_weight(p, i, dt);
    default: return 0.0;
  }
}

__device__ __forceinline__ bool is_int_dt(int dt) {
  return dt == MX_DTYPE_INT8 || dt == MX_DTYPE_INT16 || dt == MX_DTYPE_INT32 || dt == MX_DTYPE_INT64 ||
         dt == MX_DTYPE_UINT8 || dt == MX_DTYPE_UINT16 || dt == MX_DTYPE_UINT32 || dt == MX_DTYPE_UINT64 ||
         dt == MX_DTYPE_BOOL || dt == MX_DTYPE_INT4 || dt == MX_DTYPE_UINT4;
}

__device__ __forceinline__ int64_t load_as_i64(const void* p, int64_t i, int dt) {
  switch (dt) {
    case MX_DTYPE_INT8: return ((const int8_t*)p)[i];
    case MX_DTYPE_INT16: return ((const int16_t*)p)[i];
    case MX_DTYPE_INT32: return ((const int32_t*)p)[i];
    case MX_DTYPE_INT64: return ((const int64_t*)p)[i];
    case MX_DTYPE_UINT8: case MX_DTYPE_BOOL: return ((const uint8_t*)p)[i];
    case MX_DTYPE_UINT16: return ((const uint16_t*)p)[i];
    case MX_DTYPE_UINT32: return ((const uint32_t*)p)[i];
    case MX_DTYPE_UINT64: return (int64_t)((const uint64_t*)p)[i];
    case MX_DTYPE_INT4: case MX_DTYPE_UINT4: return decode_weight(p, i, dt);
    default: return (int64_t)load_as_double(p, i, dt);
  }
}

__device__ __forceinline__ void store_int(void* p, int64_t i, int dt, int64_t v) {
  switch (dt) {
    case MX_DTYPE_INT8: ((int8_t*)p)[i] = (int8_t)v; break;
    case MX_DTYPE_INT16: ((int16_t*)p)[i] = (int16_t)v; break;
    case MX_DTYPE_INT32: ((int32_t*)p)[i] = (int32_t)v; break;
    case MX_DTYPE_INT64: ((int64_t*)p)[i] = v; break;
    case MX_DTYPE_UINT8: ((uint8_t*)p)[i] = (uint8_t)v; break;
    case MX_DTYPE_BOOL: ((uint8_t*)p)[i] = v != 0; break;
    case MX_DTYPE_UINT16: ((uint16_t*)p)[i] = (uint16_t)v; break;
    case MX_DTYPE_UINT32: ((uint32_t*)p)[i] = (uint32_t)v; break;
    case MX_DTYPE_UINT64: ((uint64_t*)p)[i] = (uint64_t)v; break;
    default: break;
  }
}

// Stores an f64 value into a float dtype the way the reference does: f32 = float32(v);
// half = FromFloat32(float32(v)).
__device__ __forceinline__ void store_float(void* p, int64_t i, int dt, double v) {
  switch (dt) {
    case MX_DTYPE_FLOAT32: ((float*)p)[i] = (float)v; break;
    case MX_DTYPE_FLOAT64: ((double*)p)[i] = v; break;
    case MX_DTYPE_BFLOAT16: ((uint16_t*)p)[i] = f32_to_bf16((float)v); break;
    case MX_DTYPE_FLOAT16: ((uint16_t*)p)[i] = f32_to_f16((float)v); break;
    default: break;
  }
}

// ---------------------------------------------------------------------------------------------
// ConvertDType.
// ---------------------------------------------------------------------------------------------
__global__ void convert_kernel(const void* in, int in_dt, void* out, int out_dt, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if (is_int_dt(out_dt)) {
      if (is_int_dt(in_dt)) {
        store_int(out, i, out_dt, load_as_i64(in, i, in_dt));
      } else {
        double v = load_as_double(in, i, in_dt);
        if (out_dt == MX_DTYPE_BOOL) store_int(out, i, out_dt, v != 0.0);
        else store_int(out, i, out_dt, v != v ? 0 : (int64_t)v);  // truncation toward zero
      }
    } else if (is_int_dt(in_dt)) {
      const int64_t v = load_as_i64(in, i, in_dt);
      switch (out_dt) {
        case MX_DTYPE_FLOAT32: ((float*)out)[i] = (float)v; break;
        case MX_DTYPE_FLOAT64: ((double*)out)[i] = (double)v; break;
        case MX_DTYPE_BFLOAT16: ((uint16_t*)out)[i] = f32_to_bf16((float)v); break;
        case MX_DTYPE_FLOAT16: ((uint16_t*)out)[i] = f32_to_f16((float)v); break;
      }
    } else {
      store_float(out, i, out_dt, load_as_double(in, i, in_dt));
    }
  }
}

int ew_convert(mx_backend* b, const void* in, int in_dt, void* out, int out_dt, int64_t n) {
  if (n == 0) return MX_OK;
  return launch(b, "convert", [&] { dispatch(convert_kernel, ew_blocks(n), kEwThreads, 0, b->stream, in, in_dt, out, out_dt, n); });
}

// ---------------------------------------------------------------------------------------------
// Unary ops.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ double unary_f64(int op, double x) {
  switch (op) {
    case MX_OP_ABS: return fabs(x);
    case MX_OP_NEG: return -x;
    case MX_OP_EXP: return exp(x);
    case MX_OP_ERF: return erf(x);
    case MX_OP_TANH: return tanh(x);
    case MX_OP_SQRT: return sqrt(x);
    case MX_OP_RSQRT: return 1.0 / sqrt(x);
    case MX_OP_LOGISTIC:
      if (x >= 0) return 1.0 / (1.0 + exp(-x));
      else {
        const double e = exp(x);
        return e / (1.0 + e);
      }
    default: return x;
  }
}

__global__ void unary_kernel(int op, const void* in, void* out, int dt, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if (is_int_dt(dt)) {
      int64_t v = load_as_i64(in, i, dt);
      if (op == MX_OP_NEG) v = -v;
      else if (op == MX_OP_ABS) v = v < 0 ? -v : v;
      store_int(out, i, dt, v);
    } else if (dt == MX_DTYPE_FLOAT32 && (op == MX_OP_ABS || op == MX_OP_NEG)) {
      const float v = ((const float*)in)[i];
      ((float*)out)[i] = op == MX_OP_NEG ? -v : fabsf(v);
    } else {
      store_float(out, i, dt, unary_f64(op, load_as_double(in, i, dt)));
    }
  }
}

int ew_unary(mx_backend* b, int optype, const void* in, void* out, int dt, int64_t n) {
  if (n == 0) return MX_OK;
  return launch(b, "unary", [&] { dispatch(unary_kernel, ew_blocks(n), kEwThreads, 0, b->stream, optype, in, out, dt, n); });
}

// ---------------------------------------------------------------------------------------------
// Binary ops with size-1 broadcasting.
// ---------------------------------------------------------------------------------------------
struct BinDims {
  int64_t out[MX_MAX_RANK];
  int64_t ls[MX_MAX_RANK];  // lhs strides (0 on broadcast axes)
  int64_t rs[MX_MAX_RANK];
  int rank;
};

template <typename T>
__device__ __forceinline__ T bin_op(int op, T a, T c) {
  switch (op) {
    case MX_OP_ADD: return a + c;
    case MX_OP_SUB: return a - c;
    case MX_OP_MUL: return a * c;
    case MX_OP_DIV: return a / c;
    case MX_OP_MAX: return (a != a || c != c) ? (a != a ? a : c) : (a > c ? a : c);
    case MX_OP_MIN: return (a != a || c != c) ? (a != a ? a : c) : (a < c ? a : c);
    default: return a;
  }
}

__device__ __forceinline__ int64_t bin_op_int(int op, int64_t a, int64_t c) {
  switch (op) {
    case MX_OP_ADD: return a + c;
    case MX_OP_SUB: return a - c;
    case MX_OP_MUL: return a * c;
    case MX_OP_DIV: return c == 0 ? 0 : a / c;
    case MX_OP_MAX: return a > c ? a : c;
    case MX_OP_MIN: return a < c ? a : c;
    default: return a;
  }
}

__global__ void binary_kernel(int op, const void* lhs, const void* rhs, void* out, BinDims d, int dt, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t rem = i, li = 0, ri = 0;
    for (int a = d.rank - 1; a >= 0; --a) {
      const int64_t c = rem % d.out[a];
      rem /= d.out[a];
      li += c * d.ls[a];
      ri += c * d.rs[a];
    }
    switch (dt) {
      case MX_DTYPE_FLOAT32:
        ((float*)out)[i] = bin_op<float>(op, ((const float*)lhs)[li], ((const float*)rhs)[ri]);
        break;
      case MX_DTYPE_FLOAT64:
        ((double*)out)[i] = bin_op<double>(op, ((const double*)lhs)[li], ((const double*)rhs)[ri]);
        break;
      case MX_DTYPE_BFLOAT16:
        ((uint16_t*)out)[i] = f32_to_bf16(bin_op<float>(op, bf16_to_f32(((const uint16_t*)lhs)[li]),
                                                        bf16_to_f32(((const uint16_t*)rhs)[ri])));
        break;
      case MX_DTYPE_FLOAT16:
        ((uint16_t*)out)[i] = f32_to_f16(bin_op<float>(op, f16_to_f32(((const uint16_t*)lhs)[li]),
                                                       f16_to_f32(((const uint16_t*)rhs)[ri])));
        break;
      default:
        store_int(out, i, dt, bin_op_int(op, load_as_i64(lhs, li, dt), load_as_i64(rhs, ri, dt)));
    }
  }
}

int ew_binary(mx_backend* b, int optype, const void* lhs, const int64_t* lhs_dims, const void* rhs,
              const int64_t* rhs_dims, void* out, const int64_t* out_dims, int rank, int dt) {
  BinDims d{};
  d.rank = rank;
  int64_t n = 1, lst = 1, rst = 1;
  for (int a = rank - 1; a >= 0; --a) {
    d.out[a] = out_dims[a];
    d.ls[a] = lhs_dims[a] == 1 ? 0 : lst;
    d.rs[a] = rhs_dims[a] == 1 ? 0 : rst;
    lst *= lhs_dims[a];
    rst *= rhs_dims[a];
    n *= out_dims[a];
  }
  if (n == 0) return MX_OK;
  return launch(b, "binary", [&] { dispatch(binary_kernel, ew_blocks(n), kEwThreads, 0, b->stream, optype, lhs, rhs, out, d, dt, n); });
}

// ---------------------------------------------------------------------------------------------
// Strided gather (Transpose / BroadcastInDim / Slice).
// ---------------------------------------------------------------------------------------------
struct GatherDims {
  int64_t out[MX_MAX_RANK];
  int64_t st[MX_MAX_RANK];
  int64_t offset;
  int rank;
};

template <typename T>
__global__ void gather_kernel(const T* __restrict__ in, T* __restrict__ out, GatherDims d, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t rem = i, src = d.offset;
    for (int a = d.rank - 1; a >= 0; --a) {
      const int64_t c = rem % d.out[a];
      rem /= d.out[a];
      src += c * d.st[a];
    }
    out[i] = in[src];
  }
}

// Gathers whose innermost output axis reads contiguous input (stride 1, 64..4096 elements; the
// axis moves of DotGeneral's normalization and most transposes): one wave per output row works
// out the row's source offset once and its lanes copy the row, instead of a div/mod chain per
// element.  Shorter rows leave too many lanes idle (measured slower at 32) and stay per element.
template <typename T>
__global__ void gather_rows_kernel(const T* __restrict__ in, T* __restrict__ out, GatherDims d, int64_t rows) {
  const int lane = threadIdx.x & 63;
  const int64_t L = d.out[d.rank - 1];
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x >> 6);
  for (int64_t r = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); r < rows; r += waves) {
    int64_t rem = r, src = d.offset;
    for (int a = d.rank - 2; a >= 0; --a) {
      const int64_t c = rem % d.out[a];
      rem /= d.out[a];
      src += c * d.st[a];
    }
    const T* s = in + src;
    T* o = out + r * L;
    for (int64_t j = lane; j < L; j += 64) o[j] = s[j];
  }
}

int ew_gather_strided(mx_backend* b, const void* in, void* out, int elem_bytes, const int64_t* out_dims,
                      const int64_t* in_strides, int64_t in_offset, int rank) {
  GatherDims d{};
  d.rank = rank;
  d.offset = in_offset;
  int64_t n = 1;
  for (int a = 0; a < rank; ++a) {
    d.out[a] = out_dims[a];
    d.st[a] = in_strides[a];
    n *= out_dims[a];
  }
  if (n == 0) return MX_OK;
  hipStream_t st = b->stream;
  const int64_t L = rank > 0 ? out_dims[rank - 1] : 1;
  if (rank >= 2 && in_strides[rank - 1] == 1 && L >= 64 && L <= 4096) {
    const int64_t rows = n / L;
    const unsigned blocks = ew_blocks(rows * 64);
    switch (elem_bytes) {
      case 1: return launch(b, "gather_rows", [&] { dispatch(gather_rows_kernel<uint8_t>, blocks, kEwThreads, 0, st, (const uint8_t*)in, (uint8_t*)out, d, rows); });
      case 2: return launch(b, "gather_rows", [&] { dispatch(gather_rows_kernel<uint16_t>, blocks, kEwThreads, 0, st, (const uint16_t*)in, (uint16_t*)out, d, rows); });
      case 4: return launch(b, "gather_rows", [&] { dispatch(gather_rows_kernel<uint32_t>, blocks, kEwThreads, 0, st, (const uint32_t*)in, (uint32_t*)out, d, rows); });
      case 8: return launch(b, "gather_rows", [&] { dispatch(gather_rows_kernel<uint64_t>, blocks, kEwThreads, 0, st, (const uint64_t*)in, (uint64_t*)out, d, rows); });
      default: break;
    }
  }
  switch (elem_bytes) {
    case 1: return launch(b, "gather", [&] { dispatch(gather_kernel<uint8_t>, ew_blocks(n), kEwThreads, 0, st, (const uint8_t*)in, (uint8_t*)out, d, n); });
    case 2: return launch(b, "gather", [&] { dispatch(gather_kernel<uint16_t>, ew_blocks(n), kEwThreads, 0, st, (const uint16_t*)in, (uint16_t*)out, d, n); });
    case 4: return launch(b, "gather", [&] { dispatch(gather_kernel<uint32_t>, ew_blocks(n), kEwThreads, 0, st, (const uint32_t*)in, (uint32_t*)out, d, n); });
    case 8: return launch(b, "gather", [&] { dispatch(gather_kernel<uint64_t>, ew_blocks(n), kEwThreads, 0, st, (const uint64_t*)in, (uint64_t*)out, d, n); });
    default: return set_error(MX_ERR_NOT_IMPLEMENTED, "data movement of packed sub-byte dtypes is not implemented");
  }
}

// ---------------------------------------------------------------------------------------------
// Reductions: one workgroup per output element (tree over 256 threads, f32/f64/int64 partials).
// ---------------------------------------------------------------------------------------------
struct ReduceDims {
  int64_t keep_dims[MX_MAX_RANK];
  int64_t keep_st[MX_MAX_RANK];
  int64_t red_dims[MX_MAX_RANK];
  int64_t red_st[MX_MAX_RANK];
  int nkeep, nred;
  int64_t red_count;
};

template <typename TA>
__device__ __forceinline__ TA red_combine(int op, TA a, TA c) {
  if (op == MX_OP_REDUCE_SUM) return a + c;
  if (a != a) return a;
  if (c != c) return c;
  return a > c ? a : c;
}

template <typename TA>
__device__ __forceinline__ TA red_load(const void* in, int64_t i, int dt) {
  if constexpr (std::is_integral<TA>::value) return load_as_i64(in, i, dt);
  else return (TA)load_as_double(in, i, dt);
}

template <typename TA>
__device__ __forceinline__ TA red_init(int op);
template <>
__device__ __forceinline__ float red_init<float>(int op) { return op == MX_OP_REDUCE_SUM ? 0.0f : -INFINITY; }
template <>
__device__ __forceinline__ double red_init<double>(int op) { return op == MX_OP_REDUCE_SUM ? 0.0 : -INFINITY; }
template <>
__device__ __forceinline__ int64_t red_init<int64_t>(int op) { return op == MX_OP_REDUCE_SUM ? 0 : INT64_MIN; }

template <typename TA>
__global__ __launch_bounds__(256) void reduce_kernel(int op, const void* in, void* out, int dt, ReduceDims d) {
  __shared__ TA sh[256];
  const int64_t o = blockIdx.x;
  int64_t rem = o, base = 0;
  for (int a = d.nkeep - 1; a >= 0; --a) {
    const int64_t c = rem % d.keep_dims[a];
    rem /= d.keep_dims[a];
    base += c * d.keep_st[a];
  }
  TA acc = red_init<TA>(op);
  for (int64_t r = threadIdx.x; r < d.red_count; r += 256) {
    int64_t rr = r, off = base;
    for (int a = d.nred - 1; a >= 0; --a) {
      const int64_t c = rr % d.red_dims[a];
      rr /= d.red_dims[a];
      off += c * d.red_st[a];
    }
    acc = red_combine<TA>(op, acc, red_load<TA>(in, off, dt));
  }
  sh[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) sh[threadIdx.x] = red_combine<TA>(op, sh[threadIdx.x], sh[threadIdx.x + s]);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if constexpr (std::is_integral<TA>::value) store_int(out, o, dt, sh[0]);
    else store_float(out, o, dt, (double)sh[0]);
  }
}

int ew_reduce(mx_backend* b, int optype, const void* in, void* out, int dt, const int64_t* dims, int rank,
              uint32_t reduce_mask) {
  ReduceDims d{};
  int64_t st = 1, nout = 1;
  std::vector<int64_t> strides(rank);
  for (int a = rank - 1; a >= 0; --a) {
    strides[a] = st;
    st *= dims[a];
  }
  d.red_count = 1;
  for (int a = 0; a < rank; ++a) {
    if (reduce_mask & (1u << a)) {
      d.red_dims[d.nred] = dims[a];
      d.red_st[d.nred++] = strides[a];
      d.red_count *= dims[a];
    } else {
      d.keep_dims[d.nkeep] = dims[a];
      d.keep_st[d.nkeep++] = strides[a];
      nout *= dims[a];
    }
  }
  if (nout == 0) return MX_OK;
  if (nout > 0x7FFFFFFF) return set_error(MX_ERR_INVALID, "Reduce: too many outputs");
  hipStream_t s = b->stream;
  if (dt == MX_DTYPE_FLOAT64)
    return launch(b, "reduce", [&] { dispatch(reduce_kernel<double>, (unsigned)nout, 256, 0, s, optype, in, out, dt, d); });
  if (dtype_is_float(dt))
    return launch(b, "reduce", [&] { dispatch(reduce_kernel<float>, (unsigned)nout, 256, 0, s, optype, in, out, dt, d); });
  return launch(b, "reduce", [&] { dispatch(reduce_kernel<int64_t>, (unsigned)nout, 256, 0, s, optype, in, out, dt, d); });
}

// ---------------------------------------------------------------------------------------------
// Iota.
// ---------------------------------------------------------------------------------------------
__global__ void iota_kernel(void* out, int dt, int64_t inner, int64_t axis_dim, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = (i / inner) % axis_dim;
    if (is_int_dt(dt)) store_int(out, i, dt, v);
    else store_float(out, i, dt, (double)v);
  }
}

int ew_iota(mx_backend* b, void* out, int dt, const int64_t* dims, int rank, int axis) {
  int64_t n = 1, inner = 1;
  for (int a = 0; a < rank; ++a) n *= dims[a];
  for (int a = axis + 1; a < rank; ++a) inner *= dims[a];
  if (n == 0) return MX_OK;
  return launch(b, "iota", [&] { dispatch(iota_kernel, ew_blocks(n), kEwThreads, 0, b->stream, out, dt, inner, dims[axis], n); });
}

// ---------------------------------------------------------------------------------------------
// FusedDense epilogue (bias + activation; fusedops/dense.go:167-205) and FusedGelu (gelu.go).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ double act_f64(double x, int act) {
  switch (act) {
    case MX_ACT_GELU: return x * 0.5 * (1.0 + erf(x * (1.0 / 1.4142135623730951)));
    case MX_ACT_RELU: return x < 0 ? 0.0 : x;
    case MX_ACT_SILU: return x / (1.0 + exp(-x));
    case MX_ACT_HARDSWISH: {
      double v = x * (1.0 / 6.0) + 0.5;
      if (v != v) return v;
      v = v > 0 ? v : 0.0;
      v = v < 1 ? v : 1.0;
      return x * v;
    }
    case MX_ACT_TANH: return tanh(x);
    default: return x;
  }
}

__global__ void bias_act_kernel(const void* in, void* out, int dt, const void* bias, int64_t cols, int64_t n, int act) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t c = cols > 0 ? i % cols : 0;
    if (dt == MX_DTYPE_FLOAT64) {
      double v = ((const double*)in)[i];
      if (bias) v = v + ((const double*)bias)[c];
      ((double*)out)[i] = act_f64(v, act);
    } else {
      float v = load_f(in, i, dt);
      if (bias) v = add_rn(v, load_f(bias, c, dt));
      store_f(out, i, dt, act_ref(v, act));
    }
  }
}

int ew_bias_act(mx_backend* b, const void* in, void* out, int dt, const void* bias, int64_t rows, int64_t cols, int act) {
  const int64_t n = rows * cols;
  if (n == 0) return MX_OK;
  if (dt != MX_DTYPE_FLOAT32 && dt != MX_DTYPE_FLOAT64 && dt != MX_DTYPE_BFLOAT16)
    return set_error(MX_ERR_NOT_IMPLEMENTED, "FusedDense: dtype %s", dtype_name(dt));
  return launch(b, "bias_act", [&] { dispatch(bias_act_kernel, ew_blocks(n), kEwThreads, 0, b->stream, in, out, dt, bias, cols, n, act); });
}

__global__ void gelu_kernel(const void* in, void* out, int dt, int64_t n, int exact) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if (dt == MX_DTYPE_FLOAT64) {
      const double x = ((const double*)in)[i];
      double r;
      if (exact) r = x * 0.5 * (1.0 + erf(x * (1.0 / 1.4142135623730951)));
      else r = x * 0.5 * (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)));
      ((double*)out)[i] = r;
      continue;
    }
    const float x = dt == MX_DTYPE_FLOAT32 ? ((const float*)in)[i]
                                           : (dt == MX_DTYPE_BFLOAT16 ? bf16_to_f32(((const uint16_t*)in)[i])
                                                                      : f16_to_f32(((const uint16_t*)in)[i]));
    float r;
    if (exact) {
      r = act_ref(x, MX_ACT_GELU);
    } else {
      // x * 0.5 * (1 + float32(tanh(float64(sqrt(2/pi) * (x + 0.044715*x*x*x)))))  (gelu.go:120-126)
      const float inner = mul_rn(0.7978846f, add_rn(x, mul_rn(mul_rn(mul_rn(0.044715f, x), x), x)));
      r = mul_rn(mul_rn(x, 0.5f), add_rn(1.0f, (float)tanh((double)inner)));
    }
    if (dt == MX_DTYPE_FLOAT32) ((float*)out)[i] = r;
    else if (dt == MX_DTYPE_BFLOAT16) ((uint16_t*)out)[i] = f32_to_bf16(r);
    else ((uint16_t*)out)[i] = f32_to_f16(r);
  }
}

int ew_gelu(mx_backend* b, const void* in, void* out, int dt, int64_t n, int exact) {
  if (n == 0) return MX_OK;
  return launch(b, "gelu", [&] { dispatch(gelu_kernel, ew_blocks(n), kEwThreads, 0, b->stream, in, out, dt, n, exact); });
}

}  // namespace mx

namespace mx {

// ---------------------------------------------------------------------------------------------
// Row RMS normalisation (the graph compiler's fusion of the op chain written out in
// mxrt_internal.h).  One workgroup per row.  The sum of squares is accumulated exactly as the
// separate ReduceSum kernel accumulates it (256 threads, strided partial sums, then a tree in
// LDS), and every product and sum is rounded on its own (no contraction), so the result equals
// the unfused graph's bit for bit.
// ---------------------------------------------------------------------------------------------
// Rows of up to kRmsCached * 256 elements are read once into registers (all loads issued
// before the first use); longer rows are read twice.
constexpr int kRmsCached = 32;

__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* x, const float* c, const float* e, uint16_t* out,
                                                     int64_t D) {
  __shared__ float sh[256];
  const int64_t m = blockIdx.x;
  const uint16_t* xr = x + m * D;
  const int t = threadIdx.x;
  const bool cached = D <= (int64_t)kRmsCached * 256;
  // The row's two constants travel with the x loads (not after the reduction).
  const float cm = c[m], em = e[m];
  float v[kRmsCached];
  float acc = 0.0f;
  if (cached) {
    // Unconditional loads (clamped index) so that they are all in flight together; the values
    // past the row end are not used.
#pragma unroll
    for (int i = 0; i < kRmsCached; ++i) v[i] = bf16_to_f32(xr[min(t + 256 * (int64_t)i, D - 1)]);
#pragma unroll
    for (int i = 0; i < kRmsCached; ++i)
      if (t + 256 * (int64_t)i < D) acc = add_rn(acc, mul_rn(v[i], v[i]));
  } else {
    for (int64_t d = t; d < D; d += 256) {
      const float w = bf16_to_f32(xr[d]);
      acc = add_rn(acc, mul_rn(w, w));
    }
  }
  sh[t] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (t < s) sh[t] = add_rn(sh[t], sh[t + s]);
    __syncthreads();
  }
  const float tt = add_rn(mul_rn(sh[0], cm), em);
  const float inv = (float)(1.0 / sqrt((double)tt));
  if (cached) {
#pragma unroll
    for (int i = 0; i < kRmsCached; ++i) {
      const int64_t d = t + 256 * (int64_t)i;
      if (d < D) out[m * D + d] = f32_to_bf16(mul_rn(v[i], inv));
    }
  } else {
    for (int64_t d = t; d < D; d += 256) out[m * D + d] = f32_to_bf16(mul_rn(bf16_to_f32(xr[d]), inv));
  }
}

int ew_rmsnorm(mx_backend* b, const void* x, const void* c, const void* e, void* out, int64_t M, int64_t D) {
  if (M == 0 || D == 0) return MX_OK;
  if (M > 0x7FFFFFFF) return set_error(MX_ERR_INVALID, "RMS normalisation: too many rows");
  return launch(b, "rmsnorm", [&] {
    dispatch(rmsnorm_kernel, (unsigned)M, 256, 0, b->stream, (const uint16_t*)x, (const float*)c, (const float*)e,
             (uint16_t*)out, D);
  });
}

}  // namespace mx

// ------------------------------------------------------------------------------------------
// Read-only streaming pass (measurement): the HBM floor that a weight-streaming kernel of the
// same byte count is compared with.  Grid-stride 16-byte nontemporal loads, eight in flight per
// thread; the loaded words are folded into one value that an empty asm statement consumes, so
// no load is removed and nothing is stored.
// ------------------------------------------------------------------------------------------
namespace mx {
namespace {

typedef uint32_t sr_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kStreamUnroll = 8;

__global__ __launch_bounds__(256) void stream_read_kernel(const sr_u32x4* __restrict__ p, size_t n) {
  const size_t nt = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t h = 0;
  for (; i + (kStreamUnroll - 1) * nt < n; i += kStreamUnroll * nt) {
    sr_u32x4 v[kStreamUnroll];
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) v[u] = __builtin_nontemporal_load(p + i + u * nt);
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) h ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < n; i += nt) {
    const sr_u32x4 v = __builtin_nontemporal_load(p + i);
    h ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  asm volatile("" ::"v"(h));
}

}  // namespace
}  // namespace mx

extern "C" int mx_backend_debug_stream_read(mx_backend* b, const mx_buffer* const* bufs, int32_t nbufs,
                                            int32_t passes, int32_t workgroups) {
  mx::clear_error();
  MX_TRY(mx::check_device(b));
  if (!bufs || nbufs <= 0) return mx::set_error(MX_ERR_INVALID, "mx_backend_debug_stream_read: no buffers");
  if (passes < 0 || workgroups < 0)
    return mx::set_error(MX_ERR_INVALID, "mx_backend_debug_stream_read: negative passes or workgroups");
  for (int32_t i = 0; i < nbufs; ++i) {
    const mx_buffer* buf = bufs[i];
    if (!buf) return mx::set_error(MX_ERR_INVALID, "mx_backend_debug_stream_read: buffer %d is NULL", i);
    if (buf->finalized)
      return mx::set_error(MX_ERR_FINALIZED, "mx_backend_debug_stream_read: buffer %d is finalized", i);
    if (buf->b != b) return mx::set_error(MX_ERR_INVALID, "mx_backend_debug_stream_read: buffer %d of another backend", i);
    if ((reinterpret_cast<uintptr_t>(buf->dptr) & 15) != 0)
      return mx::set_error(MX_ERR_INVALID, "mx_backend_debug_stream_read: buffer %d not 16-byte aligned", i);
  }
  const unsigned grid = workgroups > 0 ? (unsigned)workgroups : 16u * (unsigned)std::max(b->num_cus, 1);
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  for (int32_t p = 0; p < passes; ++p) {
    const mx_buffer* buf = bufs[p % nbufs];
    const size_t n = buf->nbytes / 16;
    if (n == 0) continue;
    MX_TRY(mx::launch(b, "stream_read", [&] {
      mx::dispatch(mx::stream_read_kernel, grid, 256, 0, b->stream, (const mx::sr_u32x4*)buf->dptr, n);
    }));
  }
  return MX_OK;
}
