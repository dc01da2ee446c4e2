/*
 * mxrt.h — C ABI of the MI355X-native `compute.Backend` ("mi355x").
 *
 * This is the drop-in boundary: a Go `compute.Backend` implementation binds these entry points
 * one-to-one through cgo (every Go method of the backend is one call here).  All signatures use
 * plain C types: opaque handles, pointers, sizes and small POD structs.  No torch or HIP types
 * cross the boundary.
 *
 * Conventions (mirroring the reference's error contract, compute.go:104-115):
 *   - Every function returns an int status: MX_OK (0) or a negative MX_ERR_* code.
 *   - On error, mx_last_error() returns a thread-local, human-readable message.
 *   - MX_ERR_NOT_IMPLEMENTED is what the Go binding wraps into compute.ErrNotImplemented
 *     (compute.go:110) so callers can fall back to a decomposed graph.
 *
 * Reference citations are relative to the root of github.com/gomlx/compute.
 */
#ifndef MXRT_H_
#define MXRT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------------------------
 * Status codes.
 * ------------------------------------------------------------------------------------------- */
enum {
  MX_OK = 0,
  MX_ERR_INVALID = -1,         /* invalid argument, shape or dtype (plain error in Go)        */
  MX_ERR_NOT_IMPLEMENTED = -2, /* wraps compute.ErrNotImplemented (compute.go:110)            */
  MX_ERR_HIP = -3,             /* HIP runtime error; message carries hipGetErrorString        */
  MX_ERR_OUT_OF_MEMORY = -4,   /* device allocation failed                                    */
  MX_ERR_FINALIZED = -5,       /* use of a finalized backend/buffer/executable                */
  MX_ERR_NO_DEVICE = -6        /* backend opened host-only (graph building only), or no GPU   */
};

/* Thread-local message of the last failing call on this thread ("" if none). */
const char* mx_last_error(void);

/* ---------------------------------------------------------------------------------------------
 * Enumerations. Numeric values equal the reference's enums so the Go binding passes them through.
 * ------------------------------------------------------------------------------------------- */

/* dtypes.DType (dtypes/dtype_enum.go:20-140). Only the listed ones are accepted. */
enum {
  MX_DTYPE_INVALID = 0,
  MX_DTYPE_BOOL = 1,
  MX_DTYPE_INT8 = 2,
  MX_DTYPE_INT16 = 3,
  MX_DTYPE_INT32 = 4,
  MX_DTYPE_INT64 = 5,
  MX_DTYPE_UINT8 = 6,
  MX_DTYPE_UINT16 = 7,
  MX_DTYPE_UINT32 = 8,
  MX_DTYPE_UINT64 = 9,
  MX_DTYPE_FLOAT16 = 10,
  MX_DTYPE_FLOAT32 = 11,
  MX_DTYPE_FLOAT64 = 12,
  MX_DTYPE_BFLOAT16 = 13,
  MX_DTYPE_INT4 = 21,  /* packed, 2 per byte, low nibble first (dtypes/dtypes.go:175-239) */
  MX_DTYPE_UINT4 = 22
};

/* compute.QuantizationScheme (fused_ops.go:81-98). */
enum { MX_QUANT_LINEAR = 0, MX_QUANT_NF4 = 1, MX_QUANT_GGML = 2 };
/* compute.GGMLQuantType (fused_ops.go:134-146).  The fused paths support Q4_0, Q8_0, IQ4_NL, Q4_K
 * and Q6_K, like the reference (quantizeddense.go:145-152). */
enum {
  MX_GGML_Q4_0 = 0,
  MX_GGML_Q8_0 = 1,
  MX_GGML_IQ4_NL = 2,
  MX_GGML_Q2_K = 3,
  MX_GGML_Q3_K = 4,
  MX_GGML_Q4_K = 5,
  MX_GGML_Q5_K = 6,
  MX_GGML_Q6_K = 7
};

/* compute.ActivationType (fused_ops.go:280-289). */
enum {
  MX_ACT_NONE = 0,
  MX_ACT_GELU = 1, /* exact (erf) GELU, as the reference's fused epilogue (gelu.go:113-118) */
  MX_ACT_RELU = 2,
  MX_ACT_SILU = 3,
  MX_ACT_HARDSWISH = 4,
  MX_ACT_TANH = 5
};

/* compute.OpType values used by capability queries (optype.go:13-162, iota order). */
enum {
  MX_OP_PARAMETER = 1,
  MX_OP_CONSTANT = 2,
  MX_OP_IDENTITY = 3,
  MX_OP_ABS = 10,
  MX_OP_ADD = 11,
  MX_OP_BITCAST = 14,
  MX_OP_BROADCAST_IN_DIM = 19,
  MX_OP_CONVERT_DTYPE = 28,
  MX_OP_DIV = 30,
  MX_OP_DOT_GENERAL = 32,
  MX_OP_ERF = 39,
  MX_OP_EXP = 40,
  MX_OP_IOTA = 50,
  MX_OP_LOGISTIC = 63,
  MX_OP_MAX = 64,
  MX_OP_MIN = 65,
  MX_OP_MUL = 66,
  MX_OP_NEG = 67,
  MX_OP_REDUCE_MAX = 79,
  MX_OP_REDUCE_SUM = 82,
  MX_OP_RESHAPE = 84,
  MX_OP_RSQRT = 88,
  MX_OP_SLICE = 100,
  MX_OP_SQRT = 101,
  MX_OP_SUB = 102,
  MX_OP_TANH = 103,
  MX_OP_TRANSPOSE = 104,
  MX_OP_FUSED_GELU = 118,
  MX_OP_FUSED_DENSE = 119,
  MX_OP_FUSED_QUANTIZED_DENSE = 123,
  MX_OP_QUANTIZED_EMBEDDING_LOOKUP = 124
};

#define MX_MAX_RANK 8

/* shapes.Shape{DType, Dimensions} (shapes/shapes.go:68-84); static shapes only. */
typedef struct mx_shape {
  int32_t dtype;
  int32_t rank;
  int64_t dims[MX_MAX_RANK];
} mx_shape;

/* Opaque handles. */
typedef struct mx_backend mx_backend;
typedef struct mx_buffer mx_buffer;
typedef struct mx_builder mx_builder;
typedef struct mx_function mx_function;
typedef struct mx_executable mx_executable;

/* compute.Value (builder.go:12): opaque graph value. 0 means nil (e.g. "no bias"). A value is
 * only valid in the builder that created it; other builders reject it. */
typedef uint64_t mx_value;

/* ---------------------------------------------------------------------------------------------
 * Backend  —  compute.Backend (compute.go:68-102) and its constructor (compute.go:220-238).
 * ------------------------------------------------------------------------------------------- */

/* Constructor registered as "mi355x" (compute.go:129 Register / :220 NewWithConfig).
 * config: comma-separated options: "device=N"; "host_only" (graph building and shape checks
 * only; every device operation then fails with MX_ERR_NO_DEVICE); "nofusion" (compile graphs op
 * by op); "exact" (FusedQuantizedDense always in the reference's loop order, bit-identical to
 * quantizeddense.go:586-650 at every size).  Without "exact", decode and prefill shapes take the
 * fast kernels.  The bf16-x kernels (skinny, prefill GEMM) and the decode GEMV differ from the
 * reference only in summation order.  The prefill plans of the reference layout, f32 x, zero
 * points and NF4 (past 64 rows), and of GGML rows (past 20 rows), also round each term's weight
 * factor w*s (or w*s+zp) before the product with x, where the reference rounds (x*w)*s; they
 * stay within the f32 accumulation bound of the reference's sum.  Below the fast kernels'
 * thresholds (the decode GEMV from 2^20 weights, and past 64 rows, for widths whose packed rows
 * start mid-word, from 2^24 weights; the f32 dequantise-and-contract paths and the GGML paths
 * past four rows from 2^24 multiply-adds) problems take the reference-order kernel; the bf16-x
 * decode kernel has no threshold.  "gemv_over_gemm" (measurement only:
 * bf16 x with 17..64 rows takes the GEMV even where the prefill GEMM fits, which it otherwise
 * prefers). */
int mx_backend_new(const char* config, mx_backend** out);
/* Backend.Finalize (compute.go:95). Frees all device memory; later calls fail MX_ERR_FINALIZED. */
int mx_backend_finalize(mx_backend* b);
/* Backend.IsFinalized (compute.go:101). */
int mx_backend_is_finalized(const mx_backend* b);
/* Backend.Name (compute.go:70): writes "mi355x". */
int mx_backend_name(const mx_backend* b, char* buf, size_t buflen);
/* Backend.Description (compute.go:76). */
int mx_backend_description(const mx_backend* b, char* buf, size_t buflen);
/* Backend.NumDevices (compute.go:79). */
int mx_backend_num_devices(const mx_backend* b, int* out);
/* Backend.DeviceDescription (compute.go:82). */
int mx_backend_device_description(const mx_backend* b, int device, char* buf, size_t buflen);
/* Backend.Capabilities (compute.go:85, capabilities.go:12-39): per-op and per-dtype queries. */
int mx_backend_supports_op(const mx_backend* b, int optype, int* out);
int mx_backend_supports_dtype(const mx_backend* b, int dtype, int* out);
/* Blocks until all queued device work of the backend is done. */
int mx_backend_synchronize(mx_backend* b);

/* Per-kernel timing (hipEvent pairs around every launch on the backend's stream).  Used by the
 * benchmark harness; off by default.  Replaces the reference's klog V(1) kernel-choice logging
 * (dot.go:176-181). */
int mx_backend_set_profiling(mx_backend* b, int enabled);
/* Number of distinct kernels timed so far; then per-entry name, launch count and total ms. */
int mx_backend_profile_count(mx_backend* b, int* out);
int mx_backend_profile_entry(mx_backend* b, int i, char* name, size_t namelen, int64_t* launches,
                             double* total_ms);
int mx_backend_profile_reset(mx_backend* b);

/* Timing of a stretch of queued work (benchmark harness; no reference counterpart): begin
 * records an event on the backend's stream; end records a second one, waits for it and returns
 * the device time between them in milliseconds.  Unlike the per-launch profile, nothing is added
 * between the kernels, so back-to-back launches run as they would untimed. */
int mx_backend_region_begin(mx_backend* b);
int mx_backend_region_end(mx_backend* b, double* ms);

/* Host-side fault injection (no reference counterpart; failure-path tests): the n-th device
 * allocation from now fails with MX_ERR_OUT_OF_MEMORY (n <= 0 disables). */
int mx_backend_debug_fail_alloc_after(mx_backend* b, int n);
/* Inspection aid (no reference counterpart; tests): the device address of the static array that
 * mx_qdense_noalloc uses on this backend's GPU (NULL for a host_only backend).  Backends on one
 * GPU report the same address. */
int mx_backend_debug_noalloc_scratch(const mx_backend* b, void** out);
/* Measurement aid (no reference counterpart; benchmark harness): queues `passes` read-only
 * passes on the backend's stream, pass i over the storage of bufs[i % nbufs] (16-byte loads,
 * whole 16-byte words only; nothing is written), each with the given number of 256-thread
 * workgroups (0: 16 per CU).  A pass's duration is the HBM streaming floor for that many bytes,
 * the figure a weight-streaming kernel is priced against beside the 8 TB/s peak; rotating over
 * buffers larger together than the 256 MB Infinity Cache keeps the passes reading HBM. */
int mx_backend_debug_stream_read(mx_backend* b, const mx_buffer* const* bufs, int32_t nbufs, int32_t passes,
                                 int32_t workgroups);

/* ---------------------------------------------------------------------------------------------
 * Buffers  —  compute.DataInterface (buffer.go:45-61) and compute.Buffer (buffer.go:12-43).
 * ------------------------------------------------------------------------------------------- */

/* DataInterface.BufferFromFlatData (buffer.go:49). host_nbytes must equal the shape's storage
 * size (packed sub-byte dtypes: ceil(elements*bits/8), dtypes.go:221-239). Copies immediately. */
int mx_buffer_from_flat(mx_backend* b, int device, const void* host, size_t host_nbytes,
                        const mx_shape* shape, mx_buffer** out);
/* Buffer.ToFlatData (buffer.go:31). Waits for pending work that writes the buffer. */
int mx_buffer_to_flat(mx_buffer* buf, void* host, size_t host_nbytes);
/* Buffer.Shape (buffer.go:23). */
int mx_buffer_shape(const mx_buffer* buf, mx_shape* out);
/* Buffer.DeviceNum (buffer.go:26). */
int mx_buffer_device(const mx_buffer* buf, int* out);
/* Storage size in bytes of the buffer's shape. */
int mx_buffer_nbytes(const mx_buffer* buf, size_t* out);
/* Device address of the buffer's storage (for interop with caller-managed kernels). */
int mx_buffer_device_ptr(const mx_buffer* buf, void** out);
/* Buffer.Finalize (buffer.go:20): returns the device memory to the backend's pool; the handle
 * stays valid (every later use fails with MX_ERR_FINALIZED) until mx_buffer_destroy.
 * Finalizing twice is an error; a NULL handle is a no-op. */
int mx_buffer_finalize(mx_buffer* buf);
/* Frees the handle (finalizing first if needed): the Go binding calls it from the buffer's
 * runtime finalizer, the reference's garbage-collection path (buffer.go:17-20). */
int mx_buffer_destroy(mx_buffer* buf);
/* DataInterface.HasSharedBuffers (buffer.go:54): always 0 (device memory is not host-mapped). */
int mx_backend_has_shared_buffers(const mx_backend* b, int* out);

/* ---------------------------------------------------------------------------------------------
 * Builder / Function  —  compute.Builder (builder.go:29-82), compute.Function (function.go:23-135)
 * ------------------------------------------------------------------------------------------- */

/* Backend.Builder (compute.go:88). */
int mx_builder_new(mx_backend* b, const char* name, mx_builder** out);
/* Frees a builder that was never compiled (Compile consumes the builder). */
int mx_builder_destroy(mx_builder* bld);
/* Builder.Main (builder.go:37). The function handle is owned by the builder. */
int mx_builder_main(mx_builder* bld, mx_function** out);
/* Builder.OpShape (builder.go:55). */
int mx_builder_op_shape(mx_builder* bld, mx_value v, mx_shape* out);
/* Builder.Compile (builder.go:81). Consumes the builder (it must not be used again, whatever
 * the result). Requires Main's Return. */
int mx_builder_compile(mx_builder* bld, mx_executable** out);

/* Function.Parameter (function.go:57). Sharding is not supported (single GPU). */
int mx_fn_parameter(mx_function* fn, const char* name, const mx_shape* shape, mx_value* out);
/* Function.Constant (function.go:67): host data (storage bytes of `shape`) copied into the
 * graph; uploaded once at Compile and resident across Execute calls. */
int mx_fn_constant(mx_function* fn, const void* host, size_t host_nbytes, const mx_shape* shape,
                   mx_value* out);
/* Function.Shape (function.go:73). */
int mx_fn_shape(mx_function* fn, mx_value v, mx_shape* out);
/* Function.Return (function.go:88). */
int mx_fn_return(mx_function* fn, const mx_value* outputs, int n);

/* compute.Quantization (fused_ops.go:204-234), with one extension: block_axis = 0 means the
 * scale blocks run along K (the contracting axis), scale shape [ceil(K/block_size), N]; a
 * per-output-channel scale may then also be given as shape [N] (block_size = K).  block_axis = 1
 * is the reference's own layout, scale [K, ceil(N/block_size)] (fused_ops.go:208-229). */
typedef struct mx_quantization {
  int32_t scheme;      /* MX_QUANT_* */
  mx_value scale;
  mx_value zero_point; /* 0 = symmetric */
  int32_t block_axis;
  int32_t block_size;
  int32_t ggml_type;   /* MX_GGML_*, used only when scheme == MX_QUANT_GGML (scale, zero_point,
                          block_axis and block_size are then unused: the blocks embed them)   */
} mx_quantization;

/* FusedOps.FusedQuantizedDense (fused_ops.go:433-435; reference builder
 * internal/gobackend/fusedops/quantizeddense.go:58-142).  y = act(x @ dequant(w) + bias).
 * x: [batch..., K] float32 or bfloat16; w: [K, N] Int4/Uint4/Int8/Uint8; scale/zero_point/bias:
 * float32 or bfloat16; output dtype = x dtype.  bias may be 0.
 * GGML scheme (FusedQuantizedDenseGGML, quantizeddense.go:181-248): x [batch..., K] float32,
 * w [N, bytesPerRow] Uint8 in q->ggml_type blocks (K = bytesPerRow / bytesPerBlock *
 * valuesPerBlock), bias [N] float32 or 0, output float32; q->zero_point must be 0. */
int mx_fn_fused_quantized_dense(mx_function* fn, mx_value x, mx_value w, mx_value bias,
                                const mx_quantization* q, int activation, mx_value* out);

/* FusedOps.QuantizedEmbeddingLookup (fused_ops.go:408-409; reference builder
 * internal/gobackend/fusedops/quantizeddense.go:266-321).  data: [vocab, bytesPerRow] Uint8 in
 * q->ggml_type blocks (q->scheme must be MX_QUANT_GGML, else MX_ERR_NOT_IMPLEMENTED); indices:
 * any integer dtype, last dimension 1; output [indices dims[:-1]..., K] float32.  An index outside
 * [0, vocab) makes Execute fail (execQuantizedEmbeddingLookup, quantizeddense.go:455-499). */
int mx_fn_quantized_embedding_lookup(mx_function* fn, mx_value data, mx_value indices, const mx_quantization* q,
                                     mx_value* out);

/* StandardOps.DotGeneral (standard_ops.go:356-361), DotGeneralConfig (standard_ops.go:91-111).
 * accumulator_dtype / output_dtype may be MX_DTYPE_INVALID (= defaults). */
int mx_fn_dot_general(mx_function* fn, mx_value lhs, const int32_t* lhs_contracting, int n_lc,
                      const int32_t* lhs_batch, int n_lb, mx_value rhs,
                      const int32_t* rhs_contracting, int n_rc, const int32_t* rhs_batch, int n_rb,
                      int accumulator_dtype, int output_dtype, mx_value* out);

/* compute.DenseLayout (fused_ops.go:51-57). */
enum { MX_DENSE_LAYOUT_INPUT_OUTPUTS = 0, MX_DENSE_LAYOUT_OUTPUTS_INPUT = 1 };
/* compute.DenseConfig (fused_ops.go:73-77). */
typedef struct mx_dense_config {
  int32_t activation;    /* MX_ACT_*                                                          */
  int32_t weight_layout; /* MX_DENSE_LAYOUT_*: weight [in, out...] or [out..., in]             */
} mx_dense_config;
/* FusedOps.FusedDense (fused_ops.go:347; reference builder fusedops/dense.go:34-110):
 * y = act(x @ W + bias) for DenseLayoutInputOutputs, act(x @ W^T + bias) for
 * DenseLayoutOutputsInput.  Output dims: x's leading dims, then the weight's output dims.
 * options NULL = the zero DenseConfig (no activation, DenseLayoutInputOutputs). */
int mx_fn_fused_dense(mx_function* fn, mx_value x, mx_value weight, mx_value bias,
                      const mx_dense_config* options, mx_value* out);
/* FusedOps.FusedGelu (fused_ops.go:329). */
int mx_fn_fused_gelu(mx_function* fn, mx_value x, int exact, mx_value* out);

/* Elementwise ops: optype is one of MX_OP_ABS/NEG/EXP/ERF/LOGISTIC/RSQRT/SQRT/TANH/IDENTITY
 * (unary; standard_ops.go:134,418,421,524,577,590,741,823,830) or MX_OP_ADD/SUB/MUL/DIV/MAX/MIN
 * (binary; standard_ops.go:138,337,580,583,587,827). */
int mx_fn_unary(mx_function* fn, int optype, mx_value x, mx_value* out);
int mx_fn_binary(mx_function* fn, int optype, mx_value lhs, mx_value rhs, mx_value* out);
/* StandardOps.ConvertDType (standard_ops.go:330). */
int mx_fn_convert_dtype(mx_function* fn, mx_value x, int dtype, mx_value* out);
/* StandardOps.Reshape (standard_ops.go:722). */
int mx_fn_reshape(mx_function* fn, mx_value x, const int64_t* dims, int rank, mx_value* out);
/* StandardOps.Bitcast (standard_ops.go:214). */
int mx_fn_bitcast(mx_function* fn, mx_value x, int dtype, mx_value* out);
/* StandardOps.BroadcastInDim (standard_ops.go:254). */
int mx_fn_broadcast_in_dim(mx_function* fn, mx_value x, const mx_shape* shape,
                           const int32_t* axes, int n_axes, mx_value* out);
/* StandardOps.ReduceSum / ReduceMax (standard_ops.go:682,661); optype MX_OP_REDUCE_SUM/MAX. */
int mx_fn_reduce(mx_function* fn, int optype, mx_value x, const int32_t* axes, int n_axes,
                 mx_value* out);
/* StandardOps.Transpose (standard_ops.go:835). */
int mx_fn_transpose(mx_function* fn, mx_value x, const int32_t* perm, int rank, mx_value* out);
/* StandardOps.Iota (standard_ops.go:532). */
int mx_fn_iota(mx_function* fn, const mx_shape* shape, int axis, mx_value* out);
/* StandardOps.Slice (standard_ops.go:820); strides may be NULL (all 1). */
int mx_fn_slice(mx_function* fn, mx_value x, const int64_t* starts, const int64_t* limits,
                const int64_t* strides, int rank, mx_value* out);

/* ---------------------------------------------------------------------------------------------
 * Executable  —  compute.Executable (executable.go:10-37).
 * ------------------------------------------------------------------------------------------- */

/* Executable.Inputs (executable.go:15). */
int mx_exec_num_inputs(const mx_executable* e, int* out);
int mx_exec_input(const mx_executable* e, int i, char* name, size_t namelen, mx_shape* shape);
/* Executable.Outputs (executable.go:18). */
int mx_exec_num_outputs(const mx_executable* e, int* out);
int mx_exec_output(const mx_executable* e, int i, mx_shape* shape);
/* Executable.Execute (executable.go:36). donate may be NULL. outputs must have room for
 * mx_exec_num_outputs handles; each returned buffer is owned by the caller.  Work is queued on
 * the backend's stream; mx_buffer_to_flat / mx_backend_synchronize wait for it. */
int mx_exec_execute(mx_executable* e, mx_buffer* const* inputs, const uint8_t* donate, int n_inputs,
                    mx_buffer** outputs, int n_outputs);
/* Executable.Finalize (executable.go:12). */
int mx_exec_finalize(mx_executable* e);
/* Serving/benchmark loop: runs Execute `iters` times, call i on input set i % n_sets
 * (input_sets holds n_sets * n_inputs handles, set-major), releasing each call's outputs as
 * soon as they are queued.  Equivalent to the caller looping over Executable.Execute
 * (executable.go:36) and Buffer.Finalize (buffer.go:20) without a foreign-call round trip per
 * iteration.  Asynchronous like Execute. */
int mx_exec_execute_loop(mx_executable* e, mx_buffer* const* input_sets, int n_sets, int n_inputs,
                         int iters);
/* The operations Execute runs, in order, one per line (after compile-time fusion, e.g.
 * "RmsNorm", "FusedQuantizedDense+Mul"); parameters, constants and storage aliases are not
 * listed.  Writes at most buflen bytes including the terminating NUL.  No counterpart in the
 * reference: an inspection aid for callers and tests, like an HLO dump. */
int mx_exec_describe(const mx_executable* e, char* buf, size_t buflen);

/* ---------------------------------------------------------------------------------------------
 * Direct kernel entry point for the hot path (device pointers; no graph).  The compiled
 * Executable launches the same kernels.  Replaces the reference's node executor
 * execFusedQuantizedDense (internal/gobackend/fusedops/quantizeddense.go:330-418).
 * ------------------------------------------------------------------------------------------- */
typedef struct mx_qdense_args {
  const void* x;          /* [M, K], x_dtype                                                  */
  const void* w;          /* [K, N], w_dtype; Int4/Uint4 packed in the reference's packing     */
  const void* scale;      /* see mx_quantization                                               */
  const void* zero_point; /* same shape/dtype as scale, or NULL                                */
  const void* bias;       /* [N], bias_dtype, or NULL                                          */
  void* out;              /* [M, N], x_dtype                                                   */
  int64_t M, K, N;
  int32_t x_dtype, w_dtype, scale_dtype, zero_point_dtype, bias_dtype;
  int32_t scheme;         /* MX_QUANT_LINEAR or MX_QUANT_NF4                                   */
  int32_t block_axis;     /* 0: blocks along K, scale [ceil(K/B), N]; 1: reference [K, ceil(N/B)] */
  int32_t block_size;
  int32_t activation;     /* MX_ACT_*                                                          */
  int32_t ggml_type;      /* scheme MX_QUANT_GGML: MX_GGML_*; w is then [N, bytesPerRow] bytes,
                             x, bias and out float32, K the logical input features             */
} mx_qdense_args;

/* Launches y = act(x @ dequant(w) + bias) on the backend's stream (asynchronous). */
int mx_qdense(mx_backend* b, const mx_qdense_args* args);
/* Name of the kernel family mx_qdense would pick for these arguments ("gemv_i4_dot2", ...). */
int mx_qdense_plan(mx_backend* b, const mx_qdense_args* args, char* buf, size_t buflen);

/* mx_qdense without any device allocation. No counterpart in the reference: it is for callers
 * that cannot allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc). The split-K partial sums and arrival counters live in a static device array of
 * MX_QDENSE_NOALLOC_SCRATCH_BYTES per GPU, set up by mx_backend_new and held until the process
 * ends; a problem whose split-K needs more returns MX_ERR_INVALID before anything is launched.
 * Results are bit-identical to mx_qdense's, except for GGML rows past 20 rows, which mx_qdense
 * dequantises into an f32 copy: they run the decode GEMV once per group of four rows, and for
 * prefill GEMMs whose last partial round of tiles mx_qdense splits into two K halves (at most 128
 * tiles past a multiple of 256): those tiles are summed whole here (both within the f32
 * accumulation bound of the reference's sum). Every call on one GPU
 * shares the array, from any backend; the calls are ordered on the device (each call's stream
 * waits for the previous call's completion event), so calls from several streams or backends run
 * one after another.  Under graph capture that wait cannot be recorded: the caller must keep a
 * captured call from overlapping any other mx_qdense_noalloc call on the GPU, or the shared
 * arrival counters can be left wrong for every later call.  Launches are not recorded in the
 * backend's kernel profile. */
#define MX_QDENSE_NOALLOC_SCRATCH_BYTES (16u << 20)
int mx_qdense_noalloc(mx_backend* b, const mx_qdense_args* args);

/* QuantizedEmbeddingLookup on device pointers (the Executable launches the same kernel);
 * replaces execQuantizedEmbeddingLookup (internal/gobackend/fusedops/quantizeddense.go:455-499).
 * Waits for the launch: an index outside [0, vocab) is reported as MX_ERR_INVALID. */
typedef struct mx_qembed_args {
  const void* data;       /* [vocab, bytes_per_row] GGML blocks                                */
  const void* indices;    /* n indices of index_dtype (any integer dtype)                      */
  void* out;              /* [n, K] float32                                                    */
  int64_t vocab, bytes_per_row, n;
  int32_t index_dtype, ggml_type;
} mx_qembed_args;
int mx_quantized_embedding_lookup(mx_backend* b, const mx_qembed_args* args);

#ifdef __cplusplus
}
#endif

#endif /* MXRT_H_ */
