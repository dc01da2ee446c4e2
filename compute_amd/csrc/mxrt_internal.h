// Internal declarations shared by the runtime, the graph executor and the kernel launchers of
// the MI355X backend. Nothing here crosses the C ABI (see include/mxrt.h for that).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/mxrt.h"

namespace mx {

// ------------------------------------------------------------------------------------------
// Errors: thread-local last message + status code.
// ------------------------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define MX_CHECK_HIP(expr)                                                                  \
  do {                                                                                      \
    hipError_t e__ = (expr);                                                                \
    if (e__ != hipSuccess)                                                                  \
      return ::mx::set_error(MX_ERR_HIP, "%s failed: %s (%s:%d)", #expr,                    \
                             hipGetErrorString(e__), __FILE__, __LINE__);                   \
  } while (0)

#define MX_TRY(expr)                 \
  do {                               \
    int rc__ = (expr);               \
    if (rc__ != MX_OK) return rc__;  \
  } while (0)

// ------------------------------------------------------------------------------------------
// DTypes (values of dtypes.DType, dtypes/dtype_enum.go:20-140).
// ------------------------------------------------------------------------------------------
bool dtype_known(int dt);
const char* dtype_name(int dt);
int dtype_bits(int dt);             // 4 for Int4/Uint4, 8*size otherwise; 0 if unknown
bool dtype_is_float(int dt);        // F16, BF16, F32, F64
bool dtype_is_half(int dt);         // F16, BF16
bool dtype_is_int(int dt);          // signed/unsigned integers incl. packed
bool dtype_is_packed(int dt);       // Int4/Uint4

struct Shape {
  int dtype = MX_DTYPE_INVALID;
  std::vector<int64_t> dims;
  int rank() const { return (int)dims.size(); }
  int64_t size() const {
    int64_t n = 1;
    for (auto d : dims) n *= d;
    return n;
  }
  // Storage bytes; packed dtypes round up to whole bytes (dtypes.go:221-239).
  size_t nbytes() const {
    int64_t n = size();
    int b = dtype_bits(dtype);
    return (size_t)((n * b + 7) / 8);
  }
  bool operator==(const Shape& o) const { return dtype == o.dtype && dims == o.dims; }
  bool operator!=(const Shape& o) const { return !(*this == o); }
  std::string str() const;
};

int shape_from_c(const mx_shape* s, Shape* out);
void shape_to_c(const Shape& s, mx_shape* out);

// ------------------------------------------------------------------------------------------
// Device context.
// ------------------------------------------------------------------------------------------

// Caching allocator over hipMalloc.  All device work of a backend runs on one stream, so a
// block returned to the pool may be handed out again immediately: any later use is ordered
// after the earlier use on that stream.
class DevicePool {
 public:
  int alloc(size_t bytes, void** out);  // MX_OK or MX_ERR_OUT_OF_MEMORY / MX_ERR_HIP
  void release(void* p);
  void trim();                           // hipFree all cached blocks
  void destroy();                        // hipFree everything (backend finalize)
  int fail_after = 0;                    // fault injection: n-th alloc fails (0 = off)
  size_t bytes_in_use() const { return in_use_; }
  size_t bytes_cached() const { return cached_; }

 private:
  static size_t round_size(size_t b);
  std::unordered_map<void*, size_t> live_;         // ptr -> rounded size
  std::multimap<size_t, void*> free_;              // rounded size -> ptr
  size_t in_use_ = 0, cached_ = 0;
};

struct ProfEntry {
  int64_t launches = 0;
  double total_ms = 0.0;
};

struct PendingTiming {
  std::string name;
  hipEvent_t start, stop;
};

}  // namespace mx

struct mx_backend {
  int device = 0;
  bool host_only = false;
  bool no_fusion = false;  // "nofusion" option: compile graphs op by op
  // "exact" option: FusedQuantizedDense always in the reference's loop order (bit-identical to it)
  bool exact_qdense = false;
  bool gemv_over_gemm = false;  // measurement option: rows 17..64 stay on the GEMV where the skinny row groups or the GEMM fit
  bool finalized = false;
  hipStream_t stream = nullptr;
  std::recursive_mutex mu;
  mx::DevicePool pool;
  std::string description;
  int num_cus = 0;
  int xcds = 8;

  // Scratch for split-K partial sums and arrival counters. Counters are kept at zero between
  // launches (the last workgroup of a tile resets its counter), so the buffer is cleared only
  // when it is (re)allocated.
  void* scratch = nullptr;
  size_t scratch_bytes = 0;

  // The device's static scratch array for mx_qdense_noalloc (set up at backend creation), and
  // whether such a call is in progress: then scratch comes from that array and nothing may
  // allocate device memory.
  void* noalloc_scratch = nullptr;
  void* noalloc_order = nullptr;  // the device's call-ordering state (qdense_noalloc.hip)
  bool noalloc_active = false;

  // Profiling.
  bool profiling = false;
  std::vector<mx::PendingTiming> pending;
  std::vector<hipEvent_t> event_cache;
  std::map<std::string, mx::ProfEntry> prof;
  // mx_backend_region_begin / _end: one event pair around a stretch of queued work.
  hipEvent_t region_start = nullptr, region_stop = nullptr;
  bool region_open = false;

  int64_t live_buffers = 0;
};

struct mx_buffer {
  mx_backend* b = nullptr;
  mx::Shape shape;
  void* dptr = nullptr;
  size_t nbytes = 0;
  bool finalized = false;
};

namespace mx {

// Checks the backend can run device work.
int check_device(mx_backend* b);
// Allocate/free device memory from the backend's pool.
int dev_alloc(mx_backend* b, size_t bytes, void** out);
void dev_free(mx_backend* b, void* p);
// Ensures scratch has at least `bytes` (zero-filled on growth). Returns the device pointer.
// Inside mx_qdense_noalloc it returns the device's static array instead and never allocates.
int ensure_scratch(mx_backend* b, size_t bytes, void** out);
// Waits for the work queued on a stream: polls it for up to 2 ms (the thread keeps its core and
// returns as soon as the work is done), then blocks.
hipError_t wait_stream(hipStream_t st);
// Looks up this device's static scratch array for mx_qdense_noalloc (once per device) and keeps
// its address in b->noalloc_scratch; b->device must be current.
int noalloc_scratch_setup(mx_backend* b);

// Launch wrapper: when profiling is on, the kernel launched inside `fn` (through dispatch())
// carries a start/stop event pair that the runtime stamps with the kernel's own execution
// interval (hipExtLaunchKernel), so the recorded duration is the kernel's, as a profiler reports
// it, without the gap of separately recorded events.  Checks the launch status.
template <typename F>
int launch(mx_backend* b, const char* name, F&& fn);

struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
// The events for the launch in progress on this thread (null when not profiling).
extern thread_local LaunchEvents g_launch_events;

int timing_begin(mx_backend* b, LaunchEvents* ev);
int timing_end(mx_backend* b, const char* name, const LaunchEvents& ev);

template <typename F>
int launch(mx_backend* b, const char* name, F&& fn) {
  LaunchEvents ev;
  const bool timed = b->profiling && !b->noalloc_active;
  if (timed) MX_TRY(timing_begin(b, &ev));
  g_launch_events = ev;
  fn();
  g_launch_events = LaunchEvents{};
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(MX_ERR_HIP, "launch of %s failed: %s", name, hipGetErrorString(e));
  if (timed) MX_TRY(timing_end(b, name, ev));
  return MX_OK;
}

// Kernel launch on `st` (used inside launch()'s callback): kernel<<<grid, block, lds, st>>>(args)
// with the current profiling events attached.
template <typename... KArgs, typename... Args>
void dispatch(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t lds, hipStream_t st, Args&&... args) {
  hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, st, g_launch_events.start, g_launch_events.stop, 0u,
                        static_cast<KArgs>(args)...);
}

// ------------------------------------------------------------------------------------------
// Kernel launchers (implemented in the .hip files).
// ------------------------------------------------------------------------------------------

// Validated description of one FusedQuantizedDense call on device pointers.
struct QDenseDesc {
  const void* x;
  const void* w;
  const void* scale;
  const void* zp;
  const void* bias;
  void* out;
  int64_t M, K, N;
  int x_dt, w_dt, s_dt, zp_dt, b_dt;
  int scheme, block_axis, block_size, act;
  // Optional elementwise epilogue folded in by the graph compiler: out = t OP res, with t the
  // dense result rounded to its dtype and res a same-shape tensor (op 0 = none; MX_OP_ADD or
  // MX_OP_MUL), rounded again as the separate elementwise op would.
  const void* res = nullptr;
  int res_dt = 0, res_op = 0;
  // Pair: a second product over the same x with its own weights, scales, bias and activation
  // (same shapes and dtypes), out = round(round(act(x.w + bias)) * round(act2(x.w2 + bias2))):
  // the graph compiler's fusion of Mul(dense, dense) over one x (a gated MLP's gate and up).
  bool pair = false;
  const void* w2 = nullptr;
  const void* scale2 = nullptr;
  const void* bias2 = nullptr;
  int b2_dt = 0, act2 = 0;
  // GGML scheme: block format (MX_GGML_*) and bytes per weight row ([N, bpr] storage).
  int ggml_type = 0;
  int64_t bpr = 0;
};
int qdense_validate(const mx_qdense_args* a, QDenseDesc* d);
int qdense_plan_name(mx_backend* b, const QDenseDesc& d, std::string* name);
int qdense_run(mx_backend* b, const QDenseDesc& d);
// Decode GEMV over the reference's own layouts (qdense_gemv.hip): shape/layout check and launch.
bool qdense_gemv_fits(const QDenseDesc& d);
int qdense_gemv_run(mx_backend* b, const QDenseDesc& d, const char* name);
// Skinny-M MFMA kernel (qdense_skinny.hip): shape/layout check and launch.
bool qdense_skinny_fits(const QDenseDesc& d);
int qdense_skinny_run(mx_backend* b, const QDenseDesc& d, const char* name);
// GGML block formats (ggml.hip): FusedQuantizedDense with weights [N, bpr] bytes and f32 x/out,
// and QuantizedEmbeddingLookup.
struct GgmlDesc {
  const float* x;      // [M, K]
  const uint8_t* w;    // [N, bpr]
  const float* bias;   // [N] or null
  float* out;          // [M, N]
  int64_t M = 0, K = 0, N = 0, bpr = 0;
  int type = 0, act = 0;
  // Decode GEMV over one K segment of longer rows: x rows ldx floats apart (0: K), weight rows
  // row_stride bytes apart (0: bpr) with the segment's bpr bytes starting row_off bytes into
  // each; accumulate adds the sums to out (the earlier segments'), epilogue applies the bias and
  // activation (the last segment).
  int64_t ldx = 0, row_stride = 0, row_off = 0;
  int accumulate = 0, epilogue = 1;
};
struct GgmlEmbedDesc {
  const uint8_t* data;  // [vocab, bpr]
  const void* idx;      // n indices, idx_dt
  float* out;           // [n, K]
  int64_t vocab = 0, bpr = 0, K = 0, n = 0;
  int idx_dt = 0, type = 0;
};
int ggml_block_geometry(int type, int* vpb, int* bpb);
// Plan and launch; the backend's exact option selects the reference-order kernel at every size.
const char* ggml_plan_name(const mx_backend* b, const GgmlDesc& d);
int ggml_dense_run(mx_backend* b, const GgmlDesc& d);
int ggml_embed_run(mx_backend* b, const GgmlEmbedDesc& e);

// Prefill of the reference layout, f32 x, zero points and NF4 (qdense_refgemm.hip): the weights
// dequantised per K block into LDS, the contraction on the f32 matrix cores.
bool qdense_refgemm_fits(const QDenseDesc& d);
int qdense_refgemm_run(mx_backend* b, const QDenseDesc& d, const char* name);

// Prefill MFMA GEMM (qdense_gemm.hip): shape/layout check and launch.
bool qdense_gemm_fits(const QDenseDesc& d);
int qdense_gemm_run(mx_backend* b, const QDenseDesc& d, const char* name);

// Normalized DotGeneral: out[b, m, n] = sum_k lhs[b, m, k] * rhs[b, k, n] (or rhs[b, n, k] when
// rhs_transposed).
struct DotDesc {
  const void* lhs;
  const void* rhs;
  void* out;
  int64_t B, M, K, N;
  bool rhs_transposed;
  int in_dt, out_dt;  // F32 for half inputs (or the half dtype itself: the rounding folded in), else in_dt
};
int dot_run(mx_backend* b, const DotDesc& d);
// Half-precision DotGeneral on the matrix cores (qdense_gemm.hip).
bool dot_mfma_fits(const DotDesc& d);
int dot_mfma_run(mx_backend* b, const DotDesc& d, const char* name);

// Elementwise / data-movement kernels (elementwise.hip).
int ew_convert(mx_backend* b, const void* in, int in_dt, void* out, int out_dt, int64_t n);
int ew_unary(mx_backend* b, int optype, const void* in, void* out, int dt, int64_t n);
// Binary op with broadcasting: both operands are viewed with out's rank; a dimension of size 1
// broadcasts.  lhs_dims/rhs_dims have `rank` entries.
int ew_binary(mx_backend* b, int optype, const void* lhs, const int64_t* lhs_dims,
              const void* rhs, const int64_t* rhs_dims, void* out, const int64_t* out_dims,
              int rank, int dt);
// out = in with strided gather: out[idx] = in[sum_i idx_i * in_strides[i] + offset].  Covers
// Transpose, BroadcastInDim (stride 0) and Slice.
int ew_gather_strided(mx_backend* b, const void* in, void* out, int elem_bytes,
                      const int64_t* out_dims, const int64_t* in_strides, int64_t in_offset,
                      int rank);
// Reduction over a set of axes (reduce_mask bit i set = axis i reduced).
int ew_reduce(mx_backend* b, int optype, const void* in, void* out, int dt,
              const int64_t* dims, int rank, uint32_t reduce_mask);
int ew_iota(mx_backend* b, void* out, int dt, const int64_t* dims, int rank, int axis);
int ew_bias_act(mx_backend* b, const void* in, void* out, int dt, const void* bias, int64_t rows,
                int64_t cols, int act);
int ew_gelu(mx_backend* b, const void* in, void* out, int dt, int64_t n, int exact);
// Row RMS normalisation of bf16 x [M, D] with per-row f32 multiplier c and offset e:
// out = bf16(f32(x) * rsqrt(sum_d f32(x)^2 * c + e)), each step rounded as the separate ops
// (ConvertDType, Mul, ReduceSum, Mul, Add, Rsqrt, BroadcastInDim, Mul, ConvertDType) round it.
int ew_rmsnorm(mx_backend* b, const void* x, const void* c, const void* e, void* out, int64_t M, int64_t D);

}  // namespace mx
