// Graph building, compilation and execution of the MI355X backend.
//
// Mirrors the reference's Builder / Function / Executable contracts (builder.go:29-82,
// function.go:23-135, executable.go:10-37) with a static, single-stream executor:
//   - nodes are created in topological order (an op only takes values that already exist);
//   - Compile uploads constants once, resolves which nodes alias their input's storage
//     (Reshape, Bitcast), and computes for every owned allocation the step after which it is
//     dead;
//   - Execute validates the inputs (exec.go:176-233), takes output/intermediate storage from
//     the backend's caching pool, queues one kernel per node on the backend's stream and hands
//     the output allocations to the caller.  Device buffers stay resident across calls.
//
// Value handles are (builder serial << 32 | node index + 1), so a value from another builder is
// rejected the way the reference's VerifyAndCastValues does (internal/gobackend/function.go:257-297).

#include <algorithm>
#include <atomic>
#include <numeric>
#include <set>
#include <string>
#include <vector>

#include "mxrt_internal.h"

namespace mx {

enum class Op {
  kParameter,
  kConstant,
  kQDense,
  kDotNorm,
  kUnary,
  kBinary,
  kConvert,
  kReshape,  // alias
  kBitcast,  // alias
  kGather,   // transpose / broadcast / slice (strided gather)
  kReduce,
  kIota,
  kBiasAct,
  kGelu,
  kCopy,
  kRmsNorm,
  kQEmbed,  // fused row RMS normalisation (compile-time fusion)
};

static const char* op_name(Op op) {
  switch (op) {
    case Op::kParameter: return "Parameter";
    case Op::kConstant: return "Constant";
    case Op::kQDense: return "FusedQuantizedDense";
    case Op::kDotNorm: return "DotGeneral";
    case Op::kUnary: return "Unary";
    case Op::kBinary: return "Binary";
    case Op::kConvert: return "ConvertDType";
    case Op::kReshape: return "Reshape";
    case Op::kBitcast: return "Bitcast";
    case Op::kGather: return "Gather";
    case Op::kReduce: return "Reduce";
    case Op::kIota: return "Iota";
    case Op::kBiasAct: return "BiasActivation";
    case Op::kGelu: return "FusedGelu";
    case Op::kCopy: return "Copy";
    case Op::kRmsNorm: return "RmsNorm";
    case Op::kQEmbed: return "QuantizedEmbeddingLookup";
  }
  return "?";
}

struct Node {
  Op op;
  int optype = 0;
  Shape shape;
  std::vector<int> in;
  // Parameter.
  std::string name;
  int param_index = -1;
  // Constant.
  std::vector<uint8_t> data;
  // FusedQuantizedDense.
  int scheme = 0, block_axis = 0, block_size = 0, act = 0;
  int ggml_type = 0;
  int64_t bpr = 0;  // GGML: bytes per weight row
  bool has_zp = false, has_bias = false;
  int res_op = 0;  // elementwise op folded into the epilogue (operand = last input)
  // Pair (compile-time fusion of Mul(dense, dense) over one x): the second product's weights,
  // scales and bias follow the first's inputs.
  bool pair = false, has_bias2 = false;
  int act2 = 0;
  int64_t M = 0, K = 0, N = 0;
  // DotNorm.
  int64_t B = 0;
  bool rhs_t = false;
  // Gather / broadcast / reduce / iota.
  std::vector<int64_t> strides;
  std::vector<int64_t> in_dims;  // reduce: operand dims; binary: lhs dims
  std::vector<int64_t> in2_dims; // binary: rhs dims
  int64_t offset = 0;
  uint32_t mask = 0;
  int axis = 0;
  int flag = 0;
};

struct FunctionImpl {
  std::vector<Node> nodes;
  std::vector<int> params;
  std::vector<int> outputs;
  bool returned = false;
};

}  // namespace mx

struct mx_function {
  mx_builder* bld = nullptr;
};

struct mx_builder {
  mx_backend* b = nullptr;
  std::string name;
  uint32_t serial = 0;
  mx_function main;
  mx::FunctionImpl fn;
  bool compiled = false;
};

struct mx_executable {
  mx_backend* b = nullptr;
  std::string name;
  std::vector<mx::Node> nodes;
  std::vector<int> params;
  std::vector<int> outputs;
  std::vector<int> root;            // storage root of every node
  std::vector<std::vector<int>> free_after;  // roots to release after each node
  std::vector<bool> output_copy;    // output i must be copied (parameter/constant/duplicate)
  std::vector<void*> const_ptr;     // resident device copies of constants (by node)
  bool finalized = false;
};

namespace mx {

static std::atomic<uint32_t> g_builder_serial{1};

static inline mx_value make_value(const mx_builder* bld, int idx) {
  return ((uint64_t)bld->serial << 32) | (uint64_t)(idx + 1);
}

static int get_node(mx_builder* bld, mx_value v, const char* op, int* out) {
  if (v == 0) return set_error(MX_ERR_INVALID, "%s: nil value", op);
  uint32_t serial = (uint32_t)(v >> 32);
  int idx = (int)(uint32_t)(v & 0xFFFFFFFFu) - 1;
  if (serial != bld->serial)
    return set_error(MX_ERR_INVALID, "%s: value was created by a different builder than \"%s\"", op, bld->name.c_str());
  if (idx < 0 || idx >= (int)bld->fn.nodes.size())
    return set_error(MX_ERR_INVALID, "%s: invalid value handle", op);
  *out = idx;
  return MX_OK;
}

static int check_fn(mx_function* fn, const char* op) {
  if (!fn || !fn->bld) return set_error(MX_ERR_INVALID, "%s: function is NULL", op);
  if (fn->bld->compiled) return set_error(MX_ERR_INVALID, "%s: builder %s already compiled", op, fn->bld->name.c_str());
  if (fn->bld->fn.returned)
    return set_error(MX_ERR_INVALID, "%s: function already returned, it can no longer be modified", op);
  if (fn->bld->b->finalized) return set_error(MX_ERR_FINALIZED, "%s: backend finalized", op);
  return MX_OK;
}

static int add_node(mx_function* fn, Node n, mx_value* out) {
  if (!out) return set_error(MX_ERR_INVALID, "%s: out is NULL", op_name(n.op));
  auto& nodes = fn->bld->fn.nodes;
  if (nodes.size() >= 0x7FFFFFF0u) return set_error(MX_ERR_INVALID, "too many nodes");
  nodes.push_back(std::move(n));
  *out = make_value(fn->bld, (int)nodes.size() - 1);
  return MX_OK;
}

static const Shape& shape_of(mx_function* fn, int idx) { return fn->bld->fn.nodes[idx].shape; }

static std::vector<int64_t> row_major_strides(const std::vector<int64_t>& dims) {
  std::vector<int64_t> s(dims.size(), 1);
  for (int i = (int)dims.size() - 2; i >= 0; --i) s[i] = s[i + 1] * dims[i + 1];
  return s;
}

// Adds a strided gather: out[idx] = in[sum idx_i * strides_i + offset].
static int add_gather(mx_function* fn, int in, const Shape& out_shape, std::vector<int64_t> strides,
                      int64_t offset, int* out_idx) {
  Node n;
  n.op = Op::kGather;
  n.shape = out_shape;
  n.in = {in};
  n.strides = std::move(strides);
  n.offset = offset;
  mx_value v;
  MX_TRY(add_node(fn, std::move(n), &v));
  *out_idx = (int)fn->bld->fn.nodes.size() - 1;
  return MX_OK;
}

static int add_alias(mx_function* fn, Op op, int in, const Shape& shape, int* out_idx) {
  Node n;
  n.op = op;
  n.shape = shape;
  n.in = {in};
  mx_value v;
  MX_TRY(add_node(fn, std::move(n), &v));
  *out_idx = (int)fn->bld->fn.nodes.size() - 1;
  return MX_OK;
}

static int add_convert(mx_function* fn, int in, int dtype, int* out_idx) {
  const Shape& s = shape_of(fn, in);
  if (s.dtype == dtype) {
    *out_idx = in;
    return MX_OK;
  }
  Node n;
  n.op = Op::kConvert;
  n.shape = s;
  n.shape.dtype = dtype;
  n.in = {in};
  mx_value v;
  MX_TRY(add_node(fn, std::move(n), &v));
  *out_idx = (int)fn->bld->fn.nodes.size() - 1;
  return MX_OK;
}

// Transposes `in` so that its axes come in the order `perm` (no-op for the identity).
static int transpose_idx(mx_function* fn, int in, const std::vector<int>& perm, int* out_idx) {
  const Shape s = shape_of(fn, in);
  bool ident = true;
  for (int i = 0; i < (int)perm.size(); ++i) ident &= perm[i] == i;
  if (ident) {
    *out_idx = in;
    return MX_OK;
  }
  auto st = row_major_strides(s.dims);
  Shape o;
  o.dtype = s.dtype;
  std::vector<int64_t> strides;
  for (int p : perm) {
    o.dims.push_back(s.dims[p]);
    strides.push_back(st[p]);
  }
  return add_gather(fn, in, o, strides, 0, out_idx);
}

static int reshape_idx(mx_function* fn, int in, const std::vector<int64_t>& dims, int* out_idx) {
  const Shape s = shape_of(fn, in);
  if (s.dims == dims) {
    *out_idx = in;
    return MX_OK;
  }
  Shape o;
  o.dtype = s.dtype;
  o.dims = dims;
  return add_alias(fn, Op::kReshape, in, o, out_idx);
}

// ---------------------------------------------------------------------------------------------
// Capabilities (capabilities.go:12-39).
// ---------------------------------------------------------------------------------------------
static bool supported_op(int op) {
  switch (op) {
    case MX_OP_PARAMETER: case MX_OP_CONSTANT: case MX_OP_IDENTITY: case MX_OP_ABS: case MX_OP_ADD:
    case MX_OP_BITCAST: case MX_OP_BROADCAST_IN_DIM: case MX_OP_CONVERT_DTYPE: case MX_OP_DIV:
    case MX_OP_DOT_GENERAL: case MX_OP_ERF: case MX_OP_EXP: case MX_OP_IOTA: case MX_OP_LOGISTIC:
    case MX_OP_MAX: case MX_OP_MIN: case MX_OP_MUL: case MX_OP_NEG: case MX_OP_REDUCE_MAX:
    case MX_OP_REDUCE_SUM: case MX_OP_RESHAPE: case MX_OP_RSQRT: case MX_OP_SLICE: case MX_OP_SQRT:
    case MX_OP_SUB: case MX_OP_TANH: case MX_OP_TRANSPOSE: case MX_OP_FUSED_GELU: case MX_OP_FUSED_DENSE:
    case MX_OP_FUSED_QUANTIZED_DENSE: case MX_OP_QUANTIZED_EMBEDDING_LOOKUP:
      return true;
    default:
      return false;
  }
}

static bool is_unary(int op) {
  switch (op) {
    case MX_OP_ABS: case MX_OP_NEG: case MX_OP_EXP: case MX_OP_ERF: case MX_OP_LOGISTIC:
    case MX_OP_RSQRT: case MX_OP_SQRT: case MX_OP_TANH: case MX_OP_IDENTITY:
      return true;
    default:
      return false;
  }
}

static bool is_binary(int op) {
  switch (op) {
    case MX_OP_ADD: case MX_OP_SUB: case MX_OP_MUL: case MX_OP_DIV: case MX_OP_MAX: case MX_OP_MIN:
      return true;
    default:
      return false;
  }
}

static bool numeric_dtype(int dt) { return dtype_is_float(dt) || (dtype_is_int(dt) && !dtype_is_packed(dt)); }

}  // namespace mx

using namespace mx;

extern "C" {

int mx_backend_supports_op(const mx_backend* b, int optype, int* out) {
  clear_error();
  if (!b || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  *out = supported_op(optype) ? 1 : 0;
  return MX_OK;
}

// ---------------------------------------------------------------------------------------------
// Builder.
// ---------------------------------------------------------------------------------------------
int mx_builder_new(mx_backend* b, const char* name, mx_builder** out) {
  clear_error();
  if (!b || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  if (b->finalized) return set_error(MX_ERR_FINALIZED, "Builder: backend finalized");
  auto* bld = new mx_builder();
  bld->b = b;
  bld->name = name ? name : "";
  bld->serial = g_builder_serial.fetch_add(1);
  bld->main.bld = bld;
  *out = bld;
  return MX_OK;
}

int mx_builder_destroy(mx_builder* bld) {
  clear_error();
  delete bld;
  return MX_OK;
}

int mx_builder_main(mx_builder* bld, mx_function** out) {
  clear_error();
  if (!bld || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  if (bld->compiled) return set_error(MX_ERR_INVALID, "Main: builder already compiled");
  *out = &bld->main;
  return MX_OK;
}

int mx_builder_op_shape(mx_builder* bld, mx_value v, mx_shape* out) {
  clear_error();
  if (!bld || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  int idx;
  MX_TRY(get_node(bld, v, "OpShape", &idx));
  shape_to_c(bld->fn.nodes[idx].shape, out);
  return MX_OK;
}

int mx_fn_shape(mx_function* fn, mx_value v, mx_shape* out) {
  clear_error();
  if (!fn || !fn->bld || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  int idx;
  MX_TRY(get_node(fn->bld, v, "Shape", &idx));
  shape_to_c(fn->bld->fn.nodes[idx].shape, out);
  return MX_OK;
}

int mx_fn_parameter(mx_function* fn, const char* name, const mx_shape* shape, mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "Parameter"));
  Node n;
  n.op = Op::kParameter;
  MX_TRY(shape_from_c(shape, &n.shape));
  n.name = name ? name : "";
  for (int p : fn->bld->fn.params)
    if (fn->bld->fn.nodes[p].name == n.name && !n.name.empty())
      return set_error(MX_ERR_INVALID, "Parameter: name %s already used", n.name.c_str());
  n.param_index = (int)fn->bld->fn.params.size();
  MX_TRY(add_node(fn, std::move(n), out));
  fn->bld->fn.params.push_back((int)fn->bld->fn.nodes.size() - 1);
  return MX_OK;
}

int mx_fn_constant(mx_function* fn, const void* host, size_t host_nbytes, const mx_shape* shape, mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "Constant"));
  Node n;
  n.op = Op::kConstant;
  MX_TRY(shape_from_c(shape, &n.shape));
  if (host_nbytes != n.shape.nbytes())
    return set_error(MX_ERR_INVALID, "Constant: shape %s needs %zu bytes, got %zu", n.shape.str().c_str(),
                     n.shape.nbytes(), host_nbytes);
  if (host_nbytes && !host) return set_error(MX_ERR_INVALID, "Constant: data is NULL");
  n.data.assign((const uint8_t*)host, (const uint8_t*)host + host_nbytes);
  return add_node(fn, std::move(n), out);
}

int mx_fn_return(mx_function* fn, const mx_value* outputs, int n) {
  clear_error();
  MX_TRY(check_fn(fn, "Return"));
  if (n <= 0 || !outputs) return set_error(MX_ERR_INVALID, "Return: needs at least one output");
  std::vector<int> outs;
  for (int i = 0; i < n; ++i) {
    int idx;
    MX_TRY(get_node(fn->bld, outputs[i], "Return", &idx));
    outs.push_back(idx);
  }
  fn->bld->fn.outputs = outs;
  fn->bld->fn.returned = true;
  return MX_OK;
}

// ---------------------------------------------------------------------------------------------
// GGML block formats (reference builders: internal/gobackend/fusedops/quantizeddense.go:144-321).
// ---------------------------------------------------------------------------------------------
// validateGGMLTypeSupported + deriveGGMLK (quantizeddense.go:145-177).
static int ggml_derive_k(const char* op, int type, int64_t bytes_per_row, int64_t* K) {
  switch (type) {
    case MX_GGML_Q4_0: case MX_GGML_Q8_0: case MX_GGML_IQ4_NL: case MX_GGML_Q4_K: case MX_GGML_Q6_K: break;
    default: return set_error(MX_ERR_NOT_IMPLEMENTED, "%s: GGML type %d not supported in fused path", op, type);
  }
  int vpb, bpb;
  MX_TRY(ggml_block_geometry(type, &vpb, &bpb));
  if (bytes_per_row % bpb != 0)
    return set_error(MX_ERR_INVALID, "%s: bytesPerRow %lld not divisible by bytesPerBlock %d", op,
                     (long long)bytes_per_row, bpb);
  *K = bytes_per_row / bpb * vpb;
  return MX_OK;
}

// FusedQuantizedDenseGGML (quantizeddense.go:181-248): x [batch..., K] f32, w [N, bytesPerRow]
// Uint8, bias [N] f32; output [batch..., N] f32.
static int fused_quantized_dense_ggml(mx_function* fn, mx_value xv, mx_value wv, mx_value biasv,
                                      const mx_quantization* q, int activation, mx_value* out) {
  const char* op = "FusedQuantizedDense(GGML)";
  int x, w, bias = -1;
  MX_TRY(get_node(fn->bld, xv, op, &x));
  MX_TRY(get_node(fn->bld, wv, op, &w));
  if (biasv) MX_TRY(get_node(fn->bld, biasv, op, &bias));
  const Shape xs = shape_of(fn, x), ws = shape_of(fn, w);
  if (xs.dtype != MX_DTYPE_FLOAT32)
    return set_error(MX_ERR_INVALID, "%s: x must be float32, got %s", op, dtype_name(xs.dtype));
  if (xs.rank() < 1) return set_error(MX_ERR_INVALID, "%s: x must have rank >= 1, got %d", op, xs.rank());
  if (ws.rank() != 2 || ws.dtype != MX_DTYPE_UINT8)
    return set_error(MX_ERR_INVALID, "%s: weights must be [N, bytesPerRow] Uint8, got %s", op, ws.str().c_str());
  const int64_t N = ws.dims[0], bpr = ws.dims[1];
  int64_t K = 0;
  MX_TRY(ggml_derive_k(op, q->ggml_type, bpr, &K));
  if (xs.dims.back() != K)
    return set_error(MX_ERR_INVALID, "%s: x's last dim (%lld) must match K=%lld derived from weights", op,
                     (long long)xs.dims.back(), (long long)K);
  if (q->zero_point) return set_error(MX_ERR_INVALID, "%s: ZeroPoint must be nil for GGML scheme", op);
  if (bias >= 0) {
    const Shape bs = shape_of(fn, bias);
    if (bs.rank() != 1 || bs.dims[0] != N || bs.dtype != MX_DTYPE_FLOAT32)
      return set_error(MX_ERR_INVALID, "%s: bias must be [%lld] float32, got %s", op, (long long)N, bs.str().c_str());
  }
  if (activation < MX_ACT_NONE || activation > MX_ACT_TANH)
    return set_error(MX_ERR_INVALID, "%s: unknown activation %d", op, activation);
  Node n;
  n.op = Op::kQDense;
  n.shape.dtype = MX_DTYPE_FLOAT32;
  n.shape.dims = xs.dims;
  n.shape.dims.back() = N;
  n.in = {x, w};
  if (bias >= 0) n.in.push_back(bias);
  n.scheme = MX_QUANT_GGML;
  n.ggml_type = q->ggml_type;
  n.bpr = bpr;
  n.act = activation;
  n.has_bias = bias >= 0;
  n.K = K;
  n.N = N;
  n.M = 1;
  for (int i = 0; i + 1 < xs.rank(); ++i) n.M *= xs.dims[i];
  return add_node(fn, std::move(n), out);
}

// QuantizedEmbeddingLookup (quantizeddense.go:266-321).
int mx_fn_quantized_embedding_lookup(mx_function* fn, mx_value datav, mx_value idxv, const mx_quantization* q,
                                     mx_value* out) {
  clear_error();
  const char* op = "QuantizedEmbeddingLookup";
  MX_TRY(check_fn(fn, op));
  if (!q) return set_error(MX_ERR_INVALID, "%s: quantization is nil", op);
  if (q->scheme != MX_QUANT_GGML)
    return set_error(MX_ERR_NOT_IMPLEMENTED,
                     "%s: only QuantGGML scheme is supported, got %d -- please create a feature request if you need "
                     "support for a different quantization scheme",
                     op, q->scheme);
  int data, idx;
  MX_TRY(get_node(fn->bld, datav, op, &data));
  MX_TRY(get_node(fn->bld, idxv, op, &idx));
  const Shape ds = shape_of(fn, data), is = shape_of(fn, idx);
  if (ds.rank() != 2 || ds.dtype != MX_DTYPE_UINT8)
    return set_error(MX_ERR_INVALID, "%s: data must be [vocabSize, bytesPerRow] Uint8, got %s", op, ds.str().c_str());
  switch (is.dtype) {
    case MX_DTYPE_INT8: case MX_DTYPE_INT16: case MX_DTYPE_INT32: case MX_DTYPE_INT64:
    case MX_DTYPE_UINT8: case MX_DTYPE_UINT16: case MX_DTYPE_UINT32: case MX_DTYPE_UINT64: break;
    default: return set_error(MX_ERR_INVALID, "%s: indices must be integer, got %s", op, dtype_name(is.dtype));
  }
  if (is.rank() < 1 || is.dims.back() != 1)
    return set_error(MX_ERR_INVALID, "%s: indices last dim must be 1, got shape %s", op, is.str().c_str());
  int64_t K = 0;
  MX_TRY(ggml_derive_k(op, q->ggml_type, ds.dims[1], &K));
  Node n;
  n.op = Op::kQEmbed;
  n.shape.dtype = MX_DTYPE_FLOAT32;
  n.shape.dims = is.dims;
  n.shape.dims.back() = K;
  n.in = {data, idx};
  n.ggml_type = q->ggml_type;
  n.bpr = ds.dims[1];
  n.K = K;
  n.N = ds.dims[0];  // vocabulary size
  n.M = is.size();   // number of indices
  return add_node(fn, std::move(n), out);
}

// ---------------------------------------------------------------------------------------------
// FusedQuantizedDense (reference builder: internal/gobackend/fusedops/quantizeddense.go:58-142).
// ---------------------------------------------------------------------------------------------
int mx_fn_fused_quantized_dense(mx_function* fn, mx_value xv, mx_value wv, mx_value biasv,
                                const mx_quantization* q, int activation, mx_value* out) {
  clear_error();
  const char* op = "FusedQuantizedDense";
  MX_TRY(check_fn(fn, op));
  if (!q) return set_error(MX_ERR_INVALID, "%s: quantization is nil", op);
  if (q->scheme == MX_QUANT_GGML) return fused_quantized_dense_ggml(fn, xv, wv, biasv, q, activation, out);
  if (q->scheme != MX_QUANT_LINEAR && q->scheme != MX_QUANT_NF4)
    return set_error(MX_ERR_NOT_IMPLEMENTED, "%s: unknown quantization scheme %d", op, q->scheme);
  int x, w, s, zp = -1, bias = -1;
  MX_TRY(get_node(fn->bld, xv, op, &x));
  MX_TRY(get_node(fn->bld, wv, op, &w));
  MX_TRY(get_node(fn->bld, q->scale, op, &s));
  if (q->zero_point) MX_TRY(get_node(fn->bld, q->zero_point, op, &zp));
  if (biasv) MX_TRY(get_node(fn->bld, biasv, op, &bias));
  const Shape xs = shape_of(fn, x), ws = shape_of(fn, w), ss = shape_of(fn, s);
  if (xs.dtype != MX_DTYPE_FLOAT32 && xs.dtype != MX_DTYPE_BFLOAT16)
    return set_error(MX_ERR_NOT_IMPLEMENTED, "%s: x must be Float32 or BFloat16, got %s", op, dtype_name(xs.dtype));
  if (xs.rank() < 1) return set_error(MX_ERR_INVALID, "%s: x must have rank >= 1, got %d", op, xs.rank());
  const int64_t K = xs.dims.back();
  if (ws.rank() != 2 || ws.dims[0] != K)
    return set_error(MX_ERR_INVALID, "%s: weights must be [%lld, N], got %s", op, (long long)K, ws.str().c_str());
  switch (ws.dtype) {
    case MX_DTYPE_INT8: case MX_DTYPE_UINT8: case MX_DTYPE_INT4: case MX_DTYPE_UINT4: break;
    default:
      return set_error(MX_ERR_NOT_IMPLEMENTED, "%s: unsupported weights dtype %s", op, dtype_name(ws.dtype));
  }
  const int64_t N = ws.dims[1];
  const int64_t B = q->block_size;
  if (B < 1) return set_error(MX_ERR_INVALID, "%s: BlockSize must be >= 1, got %lld", op, (long long)B);
  if (q->block_axis == 1) {
    const int64_t nb = (N + B - 1) / B;
    if (ss.rank() != 2 || ss.dims[0] != K || ss.dims[1] != nb)
      return set_error(MX_ERR_INVALID, "%s: scales must be [%lld, %lld], got %s", op, (long long)K, (long long)nb,
                       ss.str().c_str());
  } else if (q->block_axis == 0) {
    const int64_t kb = K == 0 ? 0 : (K + B - 1) / B;
    const bool ok2 = ss.rank() == 2 && ss.dims[0] == kb && ss.dims[1] == N;
    const bool ok1 = kb == 1 && ss.rank() == 1 && ss.dims[0] == N;
    if (!ok2 && !ok1)
      return set_error(MX_ERR_INVALID, "%s: scales must be [%lld, %lld]%s, got %s", op, (long long)kb, (long long)N,
                       kb == 1 ? " (or [N] per output channel)" : "", ss.str().c_str());
  } else {
    return set_error(MX_ERR_INVALID, "%s: BlockAxis must be 0 (along K) or 1 (along N), got %d", op, q->block_axis);
  }
  if (ss.dtype != MX_DTYPE_FLOAT32 && ss.dtype != MX_DTYPE_BFLOAT16)
    return set_error(MX_ERR_NOT_IMPLEMENTED, "%s: scales must be Float32 or BFloat16, got %s", op, dtype_name(ss.dtype));
  if (zp >= 0) {
    if (q->scheme == MX_QUANT_NF4)
      return set_error(MX_ERR_INVALID, "%s: ZeroPoint must be nil for NF4 quantization scheme", op);
    const Shape zs = shape_of(fn, zp);
    if (zs.dims != ss.dims)
      return set_error(MX_ERR_INVALID, "%s: zero point shape %s must match scales %s", op, zs.str().c_str(), ss.str().c_str());
    if (zs.dtype != MX_DTYPE_FLOAT32 && zs.dtype != MX_DTYPE_BFLOAT16)
      return set_error(MX_ERR_NOT_IMPLEMENTED, "%s: zero point must be Float32 or BFloat16", op);
  }
  if (bias >= 0) {
    const Shape bs = shape_of(fn, bias);
    if (bs.rank() != 1 || bs.dims[0] != N)
      return set_error(MX_ERR_INVALID, "%s: bias must be [%lld], got %s", op, (long long)N, bs.str().c_str());
    if (bs.dtype != MX_DTYPE_FLOAT32 && bs.dtype != MX_DTYPE_BFLOAT16)
      return set_error(MX_ERR_NOT_IMPLEMENTED, "%s: bias must be Float32 or BFloat16", op);
  }
  if (activation < MX_ACT_NONE || activation > MX_ACT_TANH)
    return set_error(MX_ERR_INVALID, "%s: unknown activation %d", op, activation);
  Node n;
  n.op = Op::kQDense;
  n.shape.dtype = xs.dtype;
  n.shape.dims = xs.dims;
  n.shape.dims.back() = N;
  n.in = {x, w, s};
  if (zp >= 0) n.in.push_back(zp);
  if (bias >= 0) n.in.push_back(bias);
  n.scheme = q->scheme;
  n.block_axis = q->block_axis;
  n.block_size = q->block_size;
  n.act = activation;
  n.has_zp = zp >= 0;
  n.has_bias = bias >= 0;
  n.K = K;
  n.N = N;
  n.M = 1;
  for (int i = 0; i + 1 < xs.rank(); ++i) n.M *= xs.dims[i];
  return add_node(fn, std::move(n), out);
}

// ---------------------------------------------------------------------------------------------
// DotGeneral (shape rules: shapeinference/dotgeneral.go:16-152; lowering: dot/dot.go:165-285).
// ---------------------------------------------------------------------------------------------
static int dot_general_idx(mx_function* fn, int lhs, const int32_t* lc, int n_lc, const int32_t* lb, int n_lb, int rhs,
                           const int32_t* rc, int n_rc, const int32_t* rb, int n_rb, int acc_dt, int out_dt,
                           int* out_idx) {
  const char* op = "DotGeneral";
  const Shape ls = shape_of(fn, lhs), rs = shape_of(fn, rhs);
  if (ls.dtype != rs.dtype)
    return set_error(MX_ERR_INVALID, "DotGeneral requires inputs with the same DType, got lhs=%s and rhs=%s",
                     dtype_name(ls.dtype), dtype_name(rs.dtype));
  if (n_lc != n_rc)
    return set_error(MX_ERR_INVALID, "DotGeneral number of contracting axes for lhs (%d) doesn't match rhs (%d)", n_lc, n_rc);
  if (n_lb != n_rb)
    return set_error(MX_ERR_INVALID, "DotGeneral number of batch axes for lhs (%d) doesn't match rhs (%d)", n_lb, n_rb);
  std::vector<bool> lused(ls.rank()), rused(rs.rank());
  auto claim = [&](std::vector<bool>& used, int axis, int rank, const char* side, const char* kind) -> int {
    if (axis < 0 || axis >= rank)
      return set_error(MX_ERR_INVALID, "DotGeneral %s %s axis %d out of bounds for rank %d", side, kind, axis, rank);
    if (used[axis]) return set_error(MX_ERR_INVALID, "DotGeneral %s axis %d used more than once in contracting/batch", side, axis);
    used[axis] = true;
    return MX_OK;
  };
  for (int i = 0; i < n_lc; ++i) {
    MX_TRY(claim(lused, lc[i], ls.rank(), "lhs", "contracting"));
    MX_TRY(claim(rused, rc[i], rs.rank(), "rhs", "contracting"));
    if (ls.dims[lc[i]] != rs.dims[rc[i]])
      return set_error(MX_ERR_INVALID, "DotGeneral contracting dimensions do not match: lhs[%d]=%lld, rhs[%d]=%lld", lc[i],
                       (long long)ls.dims[lc[i]], rc[i], (long long)rs.dims[rc[i]]);
  }
  for (int i = 0; i < n_lb; ++i) {
    MX_TRY(claim(lused, lb[i], ls.rank(), "lhs", "batch"));
    MX_TRY(claim(rused, rb[i], rs.rank(), "rhs", "batch"));
    if (ls.dims[lb[i]] != rs.dims[rb[i]])
      return set_error(MX_ERR_INVALID, "DotGeneral batch dimensions do not match: lhs[%d]=%lld, rhs[%d]=%lld", lb[i],
                       (long long)ls.dims[lb[i]], rb[i], (long long)rs.dims[rb[i]]);
  }
  const int in_dt = ls.dtype;
  // Float and (unpacked) integer dtypes, like the reference's registered implementations
  // (dot/matmul/nosimd.go:66-75 for the integers); integer sums wrap in the accumulator dtype.
  auto dot_dtype = [](int dt) { return dtype_is_float(dt) || (dtype_is_int(dt) && !dtype_is_packed(dt)); };
  if (!dot_dtype(in_dt))
    return set_error(MX_ERR_NOT_IMPLEMENTED, "%s: dtype %s not implemented", op, dtype_name(in_dt));
  if (acc_dt != MX_DTYPE_INVALID && !dot_dtype(acc_dt))
    return set_error(MX_ERR_NOT_IMPLEMENTED, "%s: accumulator dtype %s not implemented", op, dtype_name(acc_dt));
  if (out_dt != MX_DTYPE_INVALID && !dot_dtype(out_dt))
    return set_error(MX_ERR_NOT_IMPLEMENTED, "%s: output dtype %s not implemented", op, dtype_name(out_dt));
  const int final_dt = out_dt != MX_DTYPE_INVALID ? out_dt : in_dt;

  // Output shape: [batch..., lhs cross..., rhs cross...].
  std::vector<int> lcross, rcross;
  for (int a = 0; a < ls.rank(); ++a) if (!lused[a]) lcross.push_back(a);
  for (int a = 0; a < rs.rank(); ++a) if (!rused[a]) rcross.push_back(a);
  Shape final_shape;
  final_shape.dtype = final_dt;
  int64_t Bsz = 1, M = 1, K = 1, N = 1;
  for (int i = 0; i < n_lb; ++i) { final_shape.dims.push_back(ls.dims[lb[i]]); Bsz *= ls.dims[lb[i]]; }
  for (int a : lcross) { final_shape.dims.push_back(ls.dims[a]); M *= ls.dims[a]; }
  for (int a : rcross) { final_shape.dims.push_back(rs.dims[a]); N *= rs.dims[a]; }
  for (int i = 0; i < n_lc; ++i) K *= ls.dims[lc[i]];

  // Accumulation dtype (dot.go:207-210, 340-372): half inputs accumulate in f32; otherwise an
  // explicit accumulator dtype converts the inputs first.
  int compute_dt = in_dt;
  if (acc_dt != MX_DTYPE_INVALID && acc_dt != in_dt && !(dtype_is_half(in_dt) && acc_dt == MX_DTYPE_FLOAT32))
    compute_dt = acc_dt;
  int l = lhs, r = rhs;
  MX_TRY(add_convert(fn, l, compute_dt, &l));
  MX_TRY(add_convert(fn, r, compute_dt, &r));

  // lhs -> [B, M, K].
  std::vector<int> lperm;
  for (int i = 0; i < n_lb; ++i) lperm.push_back(lb[i]);
  for (int a : lcross) lperm.push_back(a);
  for (int i = 0; i < n_lc; ++i) lperm.push_back(lc[i]);
  MX_TRY(transpose_idx(fn, l, lperm, &l));
  MX_TRY(reshape_idx(fn, l, {Bsz, M, K}, &l));
  // rhs -> [B, K, N] when already in that order, else [B, N, K] when that needs no copy,
  // else transposed to [B, K, N].
  std::vector<int> rperm_nt, rperm_t;
  for (int i = 0; i < n_rb; ++i) { rperm_nt.push_back(rb[i]); rperm_t.push_back(rb[i]); }
  for (int i = 0; i < n_rc; ++i) rperm_nt.push_back(rc[i]);
  for (int a : rcross) { rperm_nt.push_back(a); rperm_t.push_back(a); }
  for (int i = 0; i < n_rc; ++i) rperm_t.push_back(rc[i]);
  auto is_ident = [](const std::vector<int>& p) {
    for (int i = 0; i < (int)p.size(); ++i) if (p[i] != i) return false;
    return true;
  };
  bool rhs_t = false;
  if (is_ident(rperm_nt)) {
    MX_TRY(reshape_idx(fn, r, {Bsz, K, N}, &r));
  } else if (is_ident(rperm_t)) {
    rhs_t = true;
    MX_TRY(reshape_idx(fn, r, {Bsz, N, K}, &r));
  } else {
    MX_TRY(transpose_idx(fn, r, rperm_nt, &r));
    MX_TRY(reshape_idx(fn, r, {Bsz, K, N}, &r));
  }
  Node n;
  n.op = Op::kDotNorm;
  n.shape.dtype = dtype_is_half(compute_dt) ? MX_DTYPE_FLOAT32 : compute_dt;
  n.shape.dims = {Bsz, M, N};
  n.in = {l, r};
  n.B = Bsz;
  n.M = M;
  n.K = K;
  n.N = N;
  n.rhs_t = rhs_t;
  mx_value v;
  MX_TRY(add_node(fn, std::move(n), &v));
  int res = (int)fn->bld->fn.nodes.size() - 1;
  MX_TRY(add_convert(fn, res, final_dt, &res));
  MX_TRY(reshape_idx(fn, res, final_shape.dims, &res));
  *out_idx = res;
  return MX_OK;
}

int mx_fn_dot_general(mx_function* fn, mx_value lhsv, const int32_t* lc, int n_lc, const int32_t* lb, int n_lb,
                      mx_value rhsv, const int32_t* rc, int n_rc, const int32_t* rb, int n_rb, int acc_dt, int out_dt,
                      mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "DotGeneral"));
  if (!out) return set_error(MX_ERR_INVALID, "DotGeneral: out is NULL");
  if ((n_lc && !lc) || (n_lb && !lb) || (n_rc && !rc) || (n_rb && !rb) || n_lc < 0 || n_lb < 0 || n_rc < 0 || n_rb < 0)
    return set_error(MX_ERR_INVALID, "DotGeneral: bad axes arguments");
  int lhs, rhs;
  MX_TRY(get_node(fn->bld, lhsv, "DotGeneral", &lhs));
  MX_TRY(get_node(fn->bld, rhsv, "DotGeneral", &rhs));
  const size_t before = fn->bld->fn.nodes.size();
  int res;
  int rc_ = dot_general_idx(fn, lhs, lc, n_lc, lb, n_lb, rhs, rc, n_rc, rb, n_rb, acc_dt, out_dt, &res);
  if (rc_ != MX_OK) {
    fn->bld->fn.nodes.resize(before);  // drop partial lowering
    return rc_;
  }
  *out = make_value(fn->bld, res);
  return MX_OK;
}

// FusedDense (fused_ops.go:347, DenseConfig fused_ops.go:73-77; reference lowering
// fusedops/dense.go:34-163): DotGeneral of x's last axis with the weight's first axis
// (DenseLayoutInputOutputs, weight [in, out...]) or last axis (DenseLayoutOutputsInput, weight
// [out..., in]), plus bias, plus activation.  Output dims: x's leading dims, then the weight's
// output dims (dense.go:59-80).
int mx_fn_fused_dense(mx_function* fn, mx_value xv, mx_value wv, mx_value biasv, const mx_dense_config* options,
                      mx_value* out) {
  clear_error();
  const char* op = "FusedDense";
  MX_TRY(check_fn(fn, op));
  const int activation = options ? options->activation : MX_ACT_NONE;
  const int layout = options ? options->weight_layout : MX_DENSE_LAYOUT_INPUT_OUTPUTS;
  int x, w, bias = -1;
  MX_TRY(get_node(fn->bld, xv, op, &x));
  MX_TRY(get_node(fn->bld, wv, op, &w));
  if (biasv) MX_TRY(get_node(fn->bld, biasv, op, &bias));
  const Shape xs = shape_of(fn, x), ws = shape_of(fn, w);
  if (xs.rank() < 1 || ws.rank() < 2)
    return set_error(MX_ERR_INVALID, "%s: x must have rank >= 1 (got %d), weight must have rank >= 2 (got %d)", op,
                     xs.rank(), ws.rank());
  const int64_t in_features = xs.dims[xs.rank() - 1];
  int32_t rc0;
  int64_t cols = 1;  // output features: the weight's dims other than the contracted one
  if (layout == MX_DENSE_LAYOUT_INPUT_OUTPUTS) {
    if (in_features != ws.dims[0])
      return set_error(MX_ERR_INVALID,
                       "%s: x's last dim (%lld) must match weight's first dim (%lld) for DenseLayoutInputOutputs", op,
                       (long long)in_features, (long long)ws.dims[0]);
    rc0 = 0;
    for (int i = 1; i < ws.rank(); ++i) cols *= ws.dims[i];
  } else if (layout == MX_DENSE_LAYOUT_OUTPUTS_INPUT) {
    const int last = ws.rank() - 1;
    if (in_features != ws.dims[last])
      return set_error(MX_ERR_INVALID,
                       "%s: x's last dim (%lld) must match weight's last dim (%lld) for DenseLayoutOutputsInput", op,
                       (long long)in_features, (long long)ws.dims[last]);
    rc0 = last;
    for (int i = 0; i < last; ++i) cols *= ws.dims[i];
  } else {
    // The reference formats the layout with %v, which prints DenseLayout.String(): "unknown".
    return set_error(MX_ERR_INVALID, "%s: unknown WeightLayout unknown", op);
  }
  if (activation < MX_ACT_NONE || activation > MX_ACT_TANH)
    return set_error(MX_ERR_INVALID, "%s: unknown activation %d", op, activation);
  if (xs.dtype != MX_DTYPE_FLOAT32 && xs.dtype != MX_DTYPE_FLOAT64 && xs.dtype != MX_DTYPE_BFLOAT16)
    return set_error(MX_ERR_NOT_IMPLEMENTED, "%s: dtype %s", op, dtype_name(xs.dtype));
  const size_t before = fn->bld->fn.nodes.size();
  int32_t lc = xs.rank() - 1;
  int y;
  int rc_ = dot_general_idx(fn, x, &lc, 1, nullptr, 0, w, &rc0, 1, nullptr, 0, MX_DTYPE_INVALID, MX_DTYPE_INVALID, &y);
  if (rc_ != MX_OK) {
    fn->bld->fn.nodes.resize(before);
    return rc_;
  }
  const Shape ys = shape_of(fn, y);
  if (bias >= 0) {
    const Shape bs = shape_of(fn, bias);
    if (bs.dtype != xs.dtype || bs.size() != cols) {
      fn->bld->fn.nodes.resize(before);
      return set_error(MX_ERR_INVALID, "%s: bias %s does not match output features %lld", op, bs.str().c_str(),
                       (long long)cols);
    }
  }
  if (bias < 0 && activation == MX_ACT_NONE) {
    *out = make_value(fn->bld, y);
    return MX_OK;
  }
  Node n;
  n.op = Op::kBiasAct;
  n.shape = ys;
  n.in = {y};
  if (bias >= 0) n.in.push_back(bias);
  n.act = activation;
  n.N = cols;
  n.M = ys.size() / std::max<int64_t>(cols, 1);
  return add_node(fn, std::move(n), out);
}

int mx_fn_fused_gelu(mx_function* fn, mx_value xv, int exact, mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "FusedGelu"));
  int x;
  MX_TRY(get_node(fn->bld, xv, "FusedGelu", &x));
  const Shape xs = shape_of(fn, x);
  if (!dtype_is_float(xs.dtype)) return set_error(MX_ERR_NOT_IMPLEMENTED, "FusedGelu: dtype %s", dtype_name(xs.dtype));
  Node n;
  n.op = Op::kGelu;
  n.shape = xs;
  n.in = {x};
  n.flag = exact ? 1 : 0;
  return add_node(fn, std::move(n), out);
}

// ---------------------------------------------------------------------------------------------
// Elementwise and data movement.
// ---------------------------------------------------------------------------------------------
int mx_fn_unary(mx_function* fn, int optype, mx_value xv, mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "Unary"));
  if (!is_unary(optype)) return set_error(MX_ERR_NOT_IMPLEMENTED, "unary op type %d not implemented", optype);
  int x;
  MX_TRY(get_node(fn->bld, xv, "Unary", &x));
  const Shape xs = shape_of(fn, x);
  if (optype == MX_OP_IDENTITY) {
    Node n;
    n.op = Op::kCopy;
    n.shape = xs;
    n.in = {x};
    return add_node(fn, std::move(n), out);
  }
  const bool float_only = optype != MX_OP_ABS && optype != MX_OP_NEG;
  if (float_only ? !dtype_is_float(xs.dtype) : !numeric_dtype(xs.dtype))
    return set_error(MX_ERR_INVALID, "unary op %d: unsupported dtype %s", optype, dtype_name(xs.dtype));
  Node n;
  n.op = Op::kUnary;
  n.optype = optype;
  n.shape = xs;
  n.in = {x};
  return add_node(fn, std::move(n), out);
}

int mx_fn_binary(mx_function* fn, int optype, mx_value lv, mx_value rv, mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "Binary"));
  if (!is_binary(optype)) return set_error(MX_ERR_NOT_IMPLEMENTED, "binary op type %d not implemented", optype);
  int l, r;
  MX_TRY(get_node(fn->bld, lv, "Binary", &l));
  MX_TRY(get_node(fn->bld, rv, "Binary", &r));
  Shape ls = shape_of(fn, l), rs = shape_of(fn, r);
  if (ls.dtype != rs.dtype)
    return set_error(MX_ERR_INVALID, "data types (DType) for BinaryOp must match, got %s and %s", ls.str().c_str(),
                     rs.str().c_str());
  if (!numeric_dtype(ls.dtype)) return set_error(MX_ERR_INVALID, "BinaryOp: unsupported dtype %s", dtype_name(ls.dtype));
  // shapeinference.go:264-300: scalars broadcast; otherwise equal ranks, dims equal or 1.
  Shape os;
  std::vector<int64_t> ld, rd;
  if (ls.rank() == 0) {
    os = rs;
    ld.assign(rs.rank(), 1);
    rd = rs.dims;
  } else if (rs.rank() == 0) {
    os = ls;
    ld = ls.dims;
    rd.assign(ls.rank(), 1);
  } else {
    if (ls.rank() != rs.rank())
      return set_error(MX_ERR_INVALID, "if operands are not scalars, their rank must match for BinaryOp; got shapes %s and %s",
                       ls.str().c_str(), rs.str().c_str());
    os = ls;
    for (int a = 0; a < ls.rank(); ++a) {
      if (ls.dims[a] == rs.dims[a]) continue;
      if (ls.dims[a] == 1) os.dims[a] = rs.dims[a];
      else if (rs.dims[a] != 1)
        return set_error(MX_ERR_INVALID, "BinaryOp: incompatible dimensions for axis %d: %s and %s", a, ls.str().c_str(),
                         rs.str().c_str());
    }
    ld = ls.dims;
    rd = rs.dims;
  }
  Node n;
  n.op = Op::kBinary;
  n.optype = optype;
  n.shape = os;
  n.in = {l, r};
  n.in_dims = ld;
  n.in2_dims = rd;
  return add_node(fn, std::move(n), out);
}

int mx_fn_convert_dtype(mx_function* fn, mx_value xv, int dtype, mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "ConvertDType"));
  int x;
  MX_TRY(get_node(fn->bld, xv, "ConvertDType", &x));
  if (!dtype_known(dtype)) return set_error(MX_ERR_INVALID, "ConvertDType: unsupported dtype %d", dtype);
  const Shape xs = shape_of(fn, x);
  if (dtype_is_packed(dtype))
    return set_error(MX_ERR_NOT_IMPLEMENTED, "ConvertDType: conversion to %s not implemented", dtype_name(dtype));
  Node n;
  n.op = Op::kConvert;
  n.shape = xs;
  n.shape.dtype = dtype;
  n.in = {x};
  return add_node(fn, std::move(n), out);
}

int mx_fn_reshape(mx_function* fn, mx_value xv, const int64_t* dims, int rank, mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "Reshape"));
  int x;
  MX_TRY(get_node(fn->bld, xv, "Reshape", &x));
  if (rank < 0 || rank > MX_MAX_RANK || (rank && !dims)) return set_error(MX_ERR_INVALID, "Reshape: bad dimensions");
  Shape o;
  o.dtype = shape_of(fn, x).dtype;
  o.dims.assign(dims, dims + rank);
  for (auto d : o.dims) if (d < 0) return set_error(MX_ERR_INVALID, "Reshape: negative dimension");
  if (o.size() != shape_of(fn, x).size())
    return set_error(MX_ERR_INVALID, "Reshape: cannot reshape %s to %s (different sizes)", shape_of(fn, x).str().c_str(),
                     o.str().c_str());
  int idx;
  MX_TRY(add_alias(fn, Op::kReshape, x, o, &idx));
  *out = make_value(fn->bld, idx);
  return MX_OK;
}

// Bitcast (shapeinference.go:1604-1642): same-size dtypes keep the shape; a wider source gains
// a trailing axis; a narrower source drops its trailing axis.
int mx_fn_bitcast(mx_function* fn, mx_value xv, int dtype, mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "Bitcast"));
  int x;
  MX_TRY(get_node(fn->bld, xv, "Bitcast", &x));
  if (!dtype_known(dtype)) return set_error(MX_ERR_INVALID, "Bitcast: unsupported dtype %d", dtype);
  const Shape xs = shape_of(fn, x);
  const int sb = dtype_bits(xs.dtype), tb = dtype_bits(dtype);
  Shape o;
  o.dtype = dtype;
  if (sb == tb) {
    o.dims = xs.dims;
  } else if (sb > tb) {
    o.dims = xs.dims;
    o.dims.push_back(sb / tb);
  } else {
    if (xs.rank() == 0 || xs.dims.back() != tb / sb)
      return set_error(MX_ERR_INVALID, "Bitcast: last dimension of %s must be %d to bitcast to %s", xs.str().c_str(), tb / sb,
                       dtype_name(dtype));
    o.dims.assign(xs.dims.begin(), xs.dims.end() - 1);
  }
  if (o.rank() > MX_MAX_RANK) return set_error(MX_ERR_INVALID, "Bitcast: rank too large");
  int idx;
  MX_TRY(add_alias(fn, Op::kBitcast, x, o, &idx));
  *out = make_value(fn->bld, idx);
  return MX_OK;
}

// BroadcastInDim (shapeinference.go:583+): operand axis i maps to output axis axes[i] and must
// have the same size or size 1.
int mx_fn_broadcast_in_dim(mx_function* fn, mx_value xv, const mx_shape* shape, const int32_t* axes, int n_axes,
                           mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "BroadcastInDim"));
  int x;
  MX_TRY(get_node(fn->bld, xv, "BroadcastInDim", &x));
  Shape os;
  MX_TRY(shape_from_c(shape, &os));
  const Shape xs = shape_of(fn, x);
  if (os.dtype != xs.dtype) return set_error(MX_ERR_INVALID, "BroadcastInDim: dtype mismatch %s vs %s", xs.str().c_str(), os.str().c_str());
  if (n_axes != xs.rank() || (n_axes && !axes))
    return set_error(MX_ERR_INVALID, "BroadcastInDim: need %d broadcast axes, got %d", xs.rank(), n_axes);
  auto xst = row_major_strides(xs.dims);
  std::vector<int64_t> strides(os.rank(), 0);
  int prev = -1;
  for (int i = 0; i < n_axes; ++i) {
    int a = axes[i];
    if (a < 0 || a >= os.rank() || a <= prev)
      return set_error(MX_ERR_INVALID, "BroadcastInDim: broadcast axes must be increasing and within output rank");
    prev = a;
    if (xs.dims[i] != os.dims[a] && xs.dims[i] != 1)
      return set_error(MX_ERR_INVALID, "BroadcastInDim: operand dim %d (%lld) incompatible with output dim %d (%lld)", i,
                       (long long)xs.dims[i], a, (long long)os.dims[a]);
    strides[a] = xs.dims[i] == 1 ? 0 : xst[i];
  }
  int idx;
  MX_TRY(add_gather(fn, x, os, strides, 0, &idx));
  *out = make_value(fn->bld, idx);
  return MX_OK;
}

int mx_fn_reduce(mx_function* fn, int optype, mx_value xv, const int32_t* axes, int n_axes, mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "Reduce"));
  if (optype != MX_OP_REDUCE_SUM && optype != MX_OP_REDUCE_MAX)
    return set_error(MX_ERR_NOT_IMPLEMENTED, "reduce op type %d not implemented", optype);
  int x;
  MX_TRY(get_node(fn->bld, xv, "Reduce", &x));
  const Shape xs = shape_of(fn, x);
  if (!numeric_dtype(xs.dtype)) return set_error(MX_ERR_INVALID, "Reduce: unsupported dtype %s", dtype_name(xs.dtype));
  uint32_t mask = 0;
  if (n_axes == 0) {
    mask = (1u << xs.rank()) - 1;  // no axes: reduce everything
  } else {
    if (!axes) return set_error(MX_ERR_INVALID, "Reduce: axes is NULL");
    for (int i = 0; i < n_axes; ++i) {
      int a = axes[i];
      if (a < 0 || a >= xs.rank()) return set_error(MX_ERR_INVALID, "Reduce: axis %d out of range for %s", a, xs.str().c_str());
      if (mask & (1u << a)) return set_error(MX_ERR_INVALID, "Reduce: axis %d repeated", a);
      mask |= 1u << a;
    }
  }
  Node n;
  n.op = Op::kReduce;
  n.optype = optype;
  n.shape.dtype = xs.dtype;
  for (int a = 0; a < xs.rank(); ++a)
    if (!(mask & (1u << a))) n.shape.dims.push_back(xs.dims[a]);
  n.in = {x};
  n.in_dims = xs.dims;
  n.mask = mask;
  return add_node(fn, std::move(n), out);
}

int mx_fn_transpose(mx_function* fn, mx_value xv, const int32_t* perm, int rank, mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "Transpose"));
  int x;
  MX_TRY(get_node(fn->bld, xv, "Transpose", &x));
  const Shape xs = shape_of(fn, x);
  if (rank != xs.rank() || (rank && !perm)) return set_error(MX_ERR_INVALID, "Transpose: permutation must have rank %d", xs.rank());
  std::vector<int> p(perm, perm + rank);
  std::vector<int> chk = p;
  std::sort(chk.begin(), chk.end());
  for (int i = 0; i < rank; ++i) if (chk[i] != i) return set_error(MX_ERR_INVALID, "Transpose: invalid permutation");
  auto st = row_major_strides(xs.dims);
  Shape o;
  o.dtype = xs.dtype;
  std::vector<int64_t> strides;
  for (int a : p) {
    o.dims.push_back(xs.dims[a]);
    strides.push_back(st[a]);
  }
  int idx;
  MX_TRY(add_gather(fn, x, o, strides, 0, &idx));
  *out = make_value(fn->bld, idx);
  return MX_OK;
}

int mx_fn_iota(mx_function* fn, const mx_shape* shape, int axis, mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "Iota"));
  Node n;
  n.op = Op::kIota;
  MX_TRY(shape_from_c(shape, &n.shape));
  if (n.shape.rank() == 0 || axis < 0 || axis >= n.shape.rank())
    return set_error(MX_ERR_INVALID, "Iota: axis %d out of range for %s", axis, n.shape.str().c_str());
  if (!numeric_dtype(n.shape.dtype)) return set_error(MX_ERR_INVALID, "Iota: unsupported dtype %s", dtype_name(n.shape.dtype));
  n.axis = axis;
  return add_node(fn, std::move(n), out);
}

int mx_fn_slice(mx_function* fn, mx_value xv, const int64_t* starts, const int64_t* limits, const int64_t* strides,
                int rank, mx_value* out) {
  clear_error();
  MX_TRY(check_fn(fn, "Slice"));
  int x;
  MX_TRY(get_node(fn->bld, xv, "Slice", &x));
  const Shape xs = shape_of(fn, x);
  if (rank != xs.rank() || (rank && (!starts || !limits))) return set_error(MX_ERR_INVALID, "Slice: need %d starts/limits", xs.rank());
  auto st = row_major_strides(xs.dims);
  Shape o;
  o.dtype = xs.dtype;
  std::vector<int64_t> gs;
  int64_t off = 0;
  for (int a = 0; a < rank; ++a) {
    int64_t s = starts[a], l = limits[a], k = strides ? strides[a] : 1;
    if (k < 1 || s < 0 || l > xs.dims[a] || s > l)
      return set_error(MX_ERR_INVALID, "Slice: invalid range [%lld:%lld:%lld] for axis %d of %s", (long long)s, (long long)l,
                       (long long)k, a, xs.str().c_str());
    o.dims.push_back((l - s + k - 1) / k);
    gs.push_back(st[a] * k);
    off += s * st[a];
  }
  int idx;
  MX_TRY(add_gather(fn, x, o, gs, off, &idx));
  *out = make_value(fn->bld, idx);
  return MX_OK;
}

// ---------------------------------------------------------------------------------------------
// Compile.
// ---------------------------------------------------------------------------------------------
// ---------------------------------------------------------------------------------------------
// Compile-time fusion.  Rewrites patterns into fewer kernels with identical arithmetic (every
// intermediate is rounded exactly as the separate ops round it); nodes left without consumers
// are dropped by the liveness analysis that follows.
// ---------------------------------------------------------------------------------------------
static std::vector<int> count_uses(const FunctionImpl& f, const std::vector<Node>& nodes) {
  std::vector<int> uses(nodes.size(), 0);
  for (const Node& n : nodes)
    for (int j : n.in) ++uses[j];
  for (int o : f.outputs) ++uses[o];
  return uses;
}

static bool is_binary_op(const Node& n, int optype) { return n.op == Op::kBinary && n.optype == optype; }
// A binary node without broadcasting (both operands have the output's dims).
static bool same_shape_binary(const Node& n) { return n.in_dims == n.shape.dims && n.in2_dims == n.shape.dims; }

// FusedQuantizedDense followed by Add or Mul with a same-shape tensor: the op moves into the
// dense kernel's epilogue (the binary node becomes the dense node, the original dense node loses
// its only consumer).
static void fuse_dense_epilogues(const FunctionImpl& f, std::vector<Node>& nodes) {
  std::vector<int> uses = count_uses(f, nodes);
  for (size_t i = 0; i < nodes.size(); ++i) {
    Node& n = nodes[i];
    if (n.op != Op::kBinary || (n.optype != MX_OP_ADD && n.optype != MX_OP_MUL) || !same_shape_binary(n)) continue;
    // Prefer the later dense operand, so that the other one is computed before this node.
    int q = -1, r = -1;
    for (int side = 1; side >= 0; --side) {
      const int c = n.in[side];
      const Node& cn = nodes[c];
      if (cn.op == Op::kQDense && cn.scheme != MX_QUANT_GGML && cn.res_op == 0 && uses[c] == 1 && cn.shape == n.shape) {
        q = c;
        r = n.in[1 - side];
        break;
      }
    }
    if (q < 0) continue;
    Node fused = nodes[q];
    fused.in.push_back(r);
    fused.res_op = n.optype;
    n = fused;
    uses = count_uses(f, nodes);
  }
}

// FusedQuantizedDense whose folded Mul operand is another single-use FusedQuantizedDense over the
// same x with the same shapes, scheme and dtypes (a gated MLP's up and gate projections): both
// products run as one pair launch, out = round(round(up) * round(gate)), as the two kernels and
// the folded Mul round it.
static void fuse_dense_pairs(const FunctionImpl& f, std::vector<Node>& nodes) {
  std::vector<int> uses = count_uses(f, nodes);
  for (size_t i = 0; i < nodes.size(); ++i) {
    Node& n = nodes[i];
    if (n.op != Op::kQDense || n.scheme == MX_QUANT_GGML || n.res_op != MX_OP_MUL || n.pair || n.has_zp) continue;
    const int r = n.in.back();
    const Node& g = nodes[r];
    if (g.op != Op::kQDense || g.scheme != n.scheme || g.res_op != 0 || g.pair || g.has_zp || uses[r] != 1) continue;
    if (g.in[0] != n.in[0] || g.M != n.M || g.K != n.K || g.N != n.N || g.shape != n.shape ||
        g.block_axis != n.block_axis || g.block_size != n.block_size)
      continue;
    if (nodes[g.in[1]].shape != nodes[n.in[1]].shape || nodes[g.in[2]].shape != nodes[n.in[2]].shape) continue;
    n.in.pop_back();
    n.res_op = 0;
    n.pair = true;
    n.act2 = g.act;
    n.has_bias2 = g.has_bias;
    const std::vector<int> gin = g.in;
    n.in.push_back(gin[1]);
    n.in.push_back(gin[2]);
    if (g.has_bias) n.in.push_back(gin[3]);
    uses = count_uses(f, nodes);
  }
}

// DotGeneral over half inputs sums into f32, then ConvertDType rounds back (dot.go:340-372): when
// the f32 sum has no other use, the rounding moves into the contraction's epilogue.
static void fuse_dot_convert(const FunctionImpl& f, std::vector<Node>& nodes) {
  std::vector<int> uses = count_uses(f, nodes);
  for (size_t i = 0; i < nodes.size(); ++i) {
    Node& n = nodes[i];
    if (n.op != Op::kConvert || !dtype_is_half(n.shape.dtype)) continue;
    const int q = n.in[0];
    const Node& dn = nodes[q];
    if (dn.op != Op::kDotNorm || dn.shape.dtype != MX_DTYPE_FLOAT32 || uses[q] != 1) continue;
    if (nodes[dn.in[0]].shape.dtype != n.shape.dtype) continue;
    Node fused = dn;
    fused.shape.dtype = n.shape.dtype;
    n = fused;
    uses = count_uses(f, nodes);
  }
}

// RMS normalisation written out with standard ops (as a GoMLX model builds it):
//   xf = ConvertDType(x bf16 [M, D] -> f32); ss = ReduceSum(Mul(xf, xf), axis 1);
//   t = Add(Mul(ss, c), e) with c, e f32 [M]; inv = Rsqrt(t);
//   h = ConvertDType(Mul(xf, BroadcastInDim(inv, [M, D], axes {0})) -> bf16)
// becomes one RmsNorm(x, c, e) node (commuted operands of the Mul/Add nodes are matched too).
static void fuse_rms_norm(const FunctionImpl& f, std::vector<Node>& nodes) {
  std::vector<int> uses = count_uses(f, nodes);
  auto single = [&](int i) { return uses[i] == 1; };
  auto f32 = [&](int i) { return nodes[i].shape.dtype == MX_DTYPE_FLOAT32; };
  for (size_t hi = 0; hi < nodes.size(); ++hi) {
    const Node& h = nodes[hi];
    if (h.op != Op::kConvert || h.shape.dtype != MX_DTYPE_BFLOAT16 || h.shape.rank() != 2) continue;
    const int64_t M = h.shape.dims[0], D = h.shape.dims[1];
    const int hf = h.in[0];
    if (!is_binary_op(nodes[hf], MX_OP_MUL) || !f32(hf) || !single(hf) || !same_shape_binary(nodes[hf])) continue;
    // Mul(xf, invb) in either order.
    int xf = -1, invb = -1;
    for (int side = 0; side < 2; ++side) {
      const int a0 = nodes[hf].in[side], a1 = nodes[hf].in[1 - side];
      const Node& xn = nodes[a0];
      const Node& bn = nodes[a1];
      if (xn.op == Op::kConvert && nodes[xn.in[0]].shape.dtype == MX_DTYPE_BFLOAT16 && bn.op == Op::kGather &&
          single(a1) && bn.offset == 0 && bn.strides.size() == 2 && (bn.strides[0] == 1 || M == 1) &&
          bn.strides[1] == 0 &&
          nodes[bn.in[0]].shape.dims == std::vector<int64_t>{M}) {
        xf = a0;
        invb = a1;
        break;
      }
    }
    if (xf < 0) continue;
    const int inv = nodes[invb].in[0];
    if (nodes[inv].op != Op::kUnary || nodes[inv].optype != MX_OP_RSQRT || !f32(inv) || !single(inv)) continue;
    const int t = nodes[inv].in[0];
    if (!is_binary_op(nodes[t], MX_OP_ADD) || !single(t) || !same_shape_binary(nodes[t])) continue;
    // Add(ms, e) and Mul(ss, c), either order; ms must be the Mul, ss the ReduceSum.
    int ms = -1, e = -1;
    for (int side = 0; side < 2; ++side)
      if (is_binary_op(nodes[nodes[t].in[side]], MX_OP_MUL) && single(nodes[t].in[side])) {
        ms = nodes[t].in[side];
        e = nodes[t].in[1 - side];
        break;
      }
    if (ms < 0 || !same_shape_binary(nodes[ms])) continue;
    int ss = -1, c = -1;
    for (int side = 0; side < 2; ++side) {
      const int cand = nodes[ms].in[side];
      const Node& rn = nodes[cand];
      if (rn.op == Op::kReduce && rn.optype == MX_OP_REDUCE_SUM && single(cand) && rn.mask == 2u &&
          rn.in_dims == std::vector<int64_t>{M, D}) {
        ss = cand;
        c = nodes[ms].in[1 - side];
        break;
      }
    }
    if (ss < 0) continue;
    const int sq = nodes[ss].in[0];
    if (!is_binary_op(nodes[sq], MX_OP_MUL) || !single(sq) || nodes[sq].in[0] != xf || nodes[sq].in[1] != xf) continue;
    if (!f32(c) || !f32(e) || nodes[c].shape.dims != std::vector<int64_t>{M} ||
        nodes[e].shape.dims != std::vector<int64_t>{M})
      continue;
    Node fused;
    fused.op = Op::kRmsNorm;
    fused.shape = h.shape;
    fused.in = {nodes[xf].in[0], c, e};
    fused.M = M;
    fused.N = D;
    nodes[hi] = fused;
    uses = count_uses(f, nodes);
  }
}

int mx_builder_compile(mx_builder* bld, mx_executable** out) {
  clear_error();
  if (!bld || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  if (bld->compiled) return set_error(MX_ERR_INVALID, "Compile: builder already compiled");
  bld->compiled = true;
  if (!bld->fn.returned) return set_error(MX_ERR_INVALID, "Compile: Main function must have Return() called before compilation");
  mx_backend* b = bld->b;
  if (b->finalized) return set_error(MX_ERR_FINALIZED, "Compile: backend finalized");
  auto* e = new mx_executable();
  e->b = b;
  e->name = bld->name;
  e->nodes = std::move(bld->fn.nodes);
  e->params = bld->fn.params;
  e->outputs = bld->fn.outputs;
  if (!b->no_fusion) {
    fuse_rms_norm(bld->fn, e->nodes);
    fuse_dense_epilogues(bld->fn, e->nodes);
    fuse_dense_pairs(bld->fn, e->nodes);
    fuse_dot_convert(bld->fn, e->nodes);
  }
  const int nn = (int)e->nodes.size();

  // Storage roots: alias ops share their input's storage.
  e->root.resize(nn);
  for (int i = 0; i < nn; ++i) {
    const Node& n = e->nodes[i];
    e->root[i] = (n.op == Op::kReshape || n.op == Op::kBitcast) ? e->root[n.in[0]] : i;
  }
  // Only nodes that feed the outputs are executed; find them.
  std::vector<bool> live(nn, false);
  for (int o : e->outputs) live[o] = true;
  for (int i = nn - 1; i >= 0; --i)
    if (live[i]) for (int j : e->nodes[i].in) live[j] = true;
  for (int p : e->params) live[p] = true;
  // Output claiming.
  std::vector<bool> claimed(nn, false);
  e->output_copy.resize(e->outputs.size());
  for (size_t k = 0; k < e->outputs.size(); ++k) {
    int r = e->root[e->outputs[k]];
    Op rop = e->nodes[r].op;
    if (rop == Op::kParameter || rop == Op::kConstant || claimed[r]) {
      e->output_copy[k] = true;
    } else {
      e->output_copy[k] = false;
      claimed[r] = true;
    }
  }
  // Last use of every owned root.
  std::vector<int> last_use(nn, -1);
  for (int i = 0; i < nn; ++i) {
    if (!live[i]) continue;
    for (int j : e->nodes[i].in) last_use[e->root[j]] = std::max(last_use[e->root[j]], i);
  }
  e->free_after.assign(nn, {});
  for (int r = 0; r < nn; ++r) {
    if (!live[r] || e->root[r] != r || claimed[r]) continue;
    Op op = e->nodes[r].op;
    if (op == Op::kParameter || op == Op::kConstant) continue;
    int at = last_use[r] >= 0 ? last_use[r] : r;  // unused results die right away
    e->free_after[at].push_back(r);
  }
  // Mark dead nodes so Execute skips them.
  for (int i = 0; i < nn; ++i)
    if (!live[i]) e->nodes[i].flag |= 0x100;
  // Upload constants.
  e->const_ptr.assign(nn, nullptr);
  if (!b->host_only) {
    std::lock_guard<std::recursive_mutex> lk(b->mu);
    for (int i = 0; i < nn; ++i) {
      const Node& n = e->nodes[i];
      if (n.op != Op::kConstant || !live[i]) continue;
      void* d = nullptr;
      int rc = dev_alloc(b, n.data.size(), &d);
      if (rc == MX_OK && !n.data.empty()) {
        hipError_t he = hipMemcpyAsync(d, n.data.data(), n.data.size(), hipMemcpyHostToDevice, b->stream);
        if (he == hipSuccess) he = hipStreamSynchronize(b->stream);
        if (he != hipSuccess) rc = set_error(MX_ERR_HIP, "Compile: constant upload failed: %s", hipGetErrorString(he));
      }
      if (rc != MX_OK) {
        for (void* p : e->const_ptr) dev_free(b, p);
        delete e;
        return rc;
      }
      e->const_ptr[i] = d;
    }
  }
  *out = e;
  return MX_OK;
}

// ---------------------------------------------------------------------------------------------
// Executable.
// ---------------------------------------------------------------------------------------------
int mx_exec_num_inputs(const mx_executable* e, int* out) {
  clear_error();
  if (!e || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  *out = (int)e->params.size();
  return MX_OK;
}

int mx_exec_input(const mx_executable* e, int i, char* name, size_t namelen, mx_shape* shape) {
  clear_error();
  if (!e) return set_error(MX_ERR_INVALID, "NULL argument");
  if (i < 0 || i >= (int)e->params.size()) return set_error(MX_ERR_INVALID, "input %d out of range", i);
  const Node& n = e->nodes[e->params[i]];
  if (name && namelen) {
    size_t k = std::min(namelen - 1, n.name.size());
    memcpy(name, n.name.data(), k);
    name[k] = 0;
  }
  if (shape) shape_to_c(n.shape, shape);
  return MX_OK;
}

int mx_exec_num_outputs(const mx_executable* e, int* out) {
  clear_error();
  if (!e || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  *out = (int)e->outputs.size();
  return MX_OK;
}

int mx_exec_output(const mx_executable* e, int i, mx_shape* shape) {
  clear_error();
  if (!e || !shape) return set_error(MX_ERR_INVALID, "NULL argument");
  if (i < 0 || i >= (int)e->outputs.size()) return set_error(MX_ERR_INVALID, "output %d out of range", i);
  shape_to_c(e->nodes[e->outputs[i]].shape, shape);
  return MX_OK;
}

int mx_exec_finalize(mx_executable* e) {
  clear_error();
  if (!e) return MX_OK;
  if (e->b && !e->b->finalized) {
    std::lock_guard<std::recursive_mutex> lk(e->b->mu);
    for (void* p : e->const_ptr) dev_free(e->b, p);
  }
  delete e;
  return MX_OK;
}

}  // extern "C"

namespace mx {

// Runs one node; ptr[] holds the device address of every node computed so far.
static int run_node(mx_executable* e, int i, std::vector<void*>& ptr) {
  mx_backend* b = e->b;
  const Node& n = e->nodes[i];
  auto in = [&](int k) { return ptr[n.in[k]]; };
  auto ins = [&](int k) -> const Shape& { return e->nodes[n.in[k]].shape; };
  void* out = ptr[i];
  const int64_t count = n.shape.size();
  switch (n.op) {
    case Op::kQEmbed: {
      GgmlEmbedDesc g;
      g.data = (const uint8_t*)in(0);
      g.idx = in(1);
      g.out = (float*)out;
      g.vocab = n.N;
      g.bpr = n.bpr;
      g.K = n.K;
      g.n = n.M;
      g.idx_dt = ins(1).dtype;
      g.type = n.ggml_type;
      return ggml_embed_run(b, g);
    }
    case Op::kQDense: {
      QDenseDesc d{};
      if (n.scheme == MX_QUANT_GGML) {
        d.x = in(0);
        d.w = in(1);
        d.bias = n.has_bias ? in(2) : nullptr;
        d.out = out;
        d.M = n.M;
        d.K = n.K;
        d.N = n.N;
        d.x_dt = MX_DTYPE_FLOAT32;
        d.w_dt = MX_DTYPE_UINT8;
        d.b_dt = n.has_bias ? MX_DTYPE_FLOAT32 : 0;
        d.scheme = MX_QUANT_GGML;
        d.ggml_type = n.ggml_type;
        d.bpr = n.bpr;
        d.act = n.act;
        return qdense_run(b, d);
      }
      d.x = in(0);
      d.w = in(1);
      d.scale = in(2);
      int k = 3;
      d.zp = n.has_zp ? in(k++) : nullptr;
      d.bias = n.has_bias ? in(k) : nullptr;
      d.out = out;
      d.M = n.M;
      d.K = n.K;
      d.N = n.N;
      d.x_dt = ins(0).dtype;
      d.w_dt = ins(1).dtype;
      d.s_dt = ins(2).dtype;
      d.zp_dt = n.has_zp ? ins(3).dtype : 0;
      d.b_dt = n.has_bias ? ins(n.has_zp ? 4 : 3).dtype : 0;
      d.scheme = n.scheme;
      d.block_axis = n.block_axis;
      d.block_size = n.block_size;
      d.act = n.act;
      if (n.res_op) {
        d.res = in((int)n.in.size() - 1);
        d.res_dt = ins((int)n.in.size() - 1).dtype;
        d.res_op = n.res_op;
      }
      if (n.pair) {
        int j = 3 + (n.has_zp ? 1 : 0) + (n.has_bias ? 1 : 0);
        d.pair = true;
        d.w2 = in(j);
        d.scale2 = in(j + 1);
        d.bias2 = n.has_bias2 ? in(j + 2) : nullptr;
        d.b2_dt = n.has_bias2 ? ins(j + 2).dtype : 0;
        d.act2 = n.act2;
      }
      return qdense_run(b, d);
    }
    case Op::kDotNorm: {
      DotDesc d{};
      d.lhs = in(0);
      d.rhs = in(1);
      d.out = out;
      d.B = n.B;
      d.M = n.M;
      d.K = n.K;
      d.N = n.N;
      d.rhs_transposed = n.rhs_t;
      d.in_dt = ins(0).dtype;
      d.out_dt = n.shape.dtype;
      return dot_run(b, d);
    }
    case Op::kUnary:
      return ew_unary(b, n.optype, in(0), out, n.shape.dtype, count);
    case Op::kBinary:
      return ew_binary(b, n.optype, in(0), n.in_dims.data(), in(1), n.in2_dims.data(), out, n.shape.dims.data(),
                       n.shape.rank(), n.shape.dtype);
    case Op::kConvert:
      return ew_convert(b, in(0), ins(0).dtype, out, n.shape.dtype, count);
    case Op::kGather:
      return ew_gather_strided(b, in(0), out, dtype_bits(n.shape.dtype) / 8, n.shape.dims.data(), n.strides.data(),
                               n.offset, n.shape.rank());
    case Op::kReduce:
      return ew_reduce(b, n.optype, in(0), out, n.shape.dtype, n.in_dims.data(), (int)n.in_dims.size(), n.mask);
    case Op::kIota:
      return ew_iota(b, out, n.shape.dtype, n.shape.dims.data(), n.shape.rank(), n.axis);
    case Op::kBiasAct:
      return ew_bias_act(b, in(0), out, n.shape.dtype, n.in.size() > 1 ? in(1) : nullptr, n.M, n.N, n.act);
    case Op::kGelu:
      return ew_gelu(b, in(0), out, n.shape.dtype, count, n.flag & 1);
    case Op::kRmsNorm:
      return ew_rmsnorm(b, in(0), in(1), in(2), out, n.M, n.N);
    case Op::kCopy:
      if (n.shape.nbytes())
        MX_CHECK_HIP(hipMemcpyAsync(out, in(0), n.shape.nbytes(), hipMemcpyDeviceToDevice, b->stream));
      return MX_OK;
    default:
      return set_error(MX_ERR_INVALID, "internal: node %d (%s) is not executable", i, op_name(n.op));
  }
}

}  // namespace mx

extern "C" int mx_exec_describe(const mx_executable* e, char* buf, size_t buflen) {
  clear_error();
  if (!e || !buf || buflen == 0) return set_error(MX_ERR_INVALID, "Describe: NULL argument");
  std::string s;
  for (const Node& n : e->nodes) {
    if (n.flag & 0x100) continue;  // dead
    if (n.op == Op::kParameter || n.op == Op::kConstant || n.op == Op::kReshape || n.op == Op::kBitcast) continue;
    s += op_name(n.op);
    if (n.op == Op::kQDense && n.res_op) s += n.res_op == MX_OP_MUL ? "+Mul" : "+Add";
    if (n.op == Op::kQDense && n.pair) s += "+Pair";
    s += "\n";
  }
  const size_t k = std::min(buflen - 1, s.size());
  memcpy(buf, s.data(), k);
  buf[k] = 0;
  return MX_OK;
}

extern "C" int mx_exec_execute(mx_executable* e, mx_buffer* const* inputs, const uint8_t* donate, int n_inputs,
                               mx_buffer** outputs, int n_outputs) {
  clear_error();
  if (!e) return set_error(MX_ERR_INVALID, "Execute: executable is NULL");
  mx_backend* b = e->b;
  MX_TRY(check_device(b));
  if (n_inputs != (int)e->params.size())
    return set_error(MX_ERR_INVALID, "Execute: expected %d inputs, got %d", (int)e->params.size(), n_inputs);
  if (n_outputs != (int)e->outputs.size() || (n_outputs && !outputs))
    return set_error(MX_ERR_INVALID, "Execute: expected room for %d outputs, got %d", (int)e->outputs.size(), n_outputs);
  for (int i = 0; i < n_inputs; ++i) {
    const mx_buffer* in = inputs ? inputs[i] : nullptr;
    const Node& p = e->nodes[e->params[i]];
    if (!in) return set_error(MX_ERR_INVALID, "Execute: input buffer #%d is nil!?", i);
    if (in->finalized)
      return set_error(MX_ERR_INVALID, "Execute: input buffer #%d is not valid, likely it is being used after being released", i);
    if (in->b != b) return set_error(MX_ERR_INVALID, "Execute: input buffer #%d is not from this backend", i);
    if (in->shape.dims != p.shape.dims)
      return set_error(MX_ERR_INVALID, "Execute: parameter \"%s\" (input #%d) for \"%s\": expected shape %s, got %s",
                       p.name.c_str(), i, e->name.c_str(), p.shape.str().c_str(), in->shape.str().c_str());
    if (in->shape.dtype != p.shape.dtype)
      return set_error(MX_ERR_INVALID, "Execute: parameter \"%s\" (input #%d) for \"%s\": expected DType %s, got %s",
                       p.name.c_str(), i, e->name.c_str(), dtype_name(p.shape.dtype), dtype_name(in->shape.dtype));
  }
  for (int i = 0; i < n_outputs; ++i) outputs[i] = nullptr;

  std::lock_guard<std::recursive_mutex> lk(b->mu);
  MX_CHECK_HIP(hipSetDevice(b->device));
  const int nn = (int)e->nodes.size();
  std::vector<void*> ptr(nn, nullptr);
  std::vector<void*> owned;  // allocations made by this call that are not yet freed or claimed
  auto fail = [&](int rc) {
    for (void* p : owned) dev_free(b, p);
    return rc;
  };
  for (int i = 0; i < nn; ++i) {
    const Node& n = e->nodes[i];
    if (n.flag & 0x100) continue;  // not needed by any output
    if (n.op == Op::kParameter) {
      ptr[i] = inputs[n.param_index]->dptr;
      continue;
    }
    if (n.op == Op::kConstant) {
      ptr[i] = e->const_ptr[i];
      continue;
    }
    if (n.op == Op::kReshape || n.op == Op::kBitcast) {
      ptr[i] = ptr[n.in[0]];
      continue;
    }
    void* d = nullptr;
    int rc = dev_alloc(b, n.shape.nbytes(), &d);
    if (rc != MX_OK) return fail(rc);
    owned.push_back(d);
    ptr[i] = d;
    rc = run_node(e, i, ptr);
    if (rc != MX_OK) return fail(rc);
    for (int r : e->free_after[i]) {
      dev_free(b, ptr[r]);
      owned.erase(std::find(owned.begin(), owned.end(), ptr[r]));
    }
  }
  // Outputs.
  std::vector<mx_buffer*> outs(n_outputs, nullptr);
  for (int k = 0; k < n_outputs; ++k) {
    const int o = e->outputs[k];
    const Node& n = e->nodes[o];
    void* d = ptr[e->root[o]];
    if (e->output_copy[k]) {
      void* c = nullptr;
      int rc = dev_alloc(b, n.shape.nbytes(), &c);
      if (rc != MX_OK) {
        for (auto* ob : outs) if (ob) { dev_free(b, ob->dptr); delete ob; }
        return fail(rc);
      }
      if (n.shape.nbytes()) {
        hipError_t he = hipMemcpyAsync(c, d, n.shape.nbytes(), hipMemcpyDeviceToDevice, b->stream);
        if (he != hipSuccess) {
          dev_free(b, c);
          for (auto* ob : outs) if (ob) { dev_free(b, ob->dptr); delete ob; }
          return fail(set_error(MX_ERR_HIP, "Execute: output copy failed: %s", hipGetErrorString(he)));
        }
      }
      d = c;
    } else {
      owned.erase(std::find(owned.begin(), owned.end(), d));
    }
    auto* ob = new mx_buffer();
    ob->b = b;
    ob->shape = n.shape;
    ob->dptr = d;
    ob->nbytes = n.shape.nbytes();
    outs[k] = ob;
  }
  for (void* p : owned) dev_free(b, p);  // nothing should remain, but never leak
  for (int k = 0; k < n_outputs; ++k) {
    outputs[k] = outs[k];
    b->live_buffers++;
  }
  // Donated inputs become invalid after the call (executable.go:20-36); their memory returns
  // to the pool, ordered after this call's kernels on the stream.
  if (donate) {
    for (int i = 0; i < n_inputs; ++i)
      if (donate[i] && !inputs[i]->finalized) MX_TRY(mx_buffer_finalize(inputs[i]));
  }
  return MX_OK;
}

extern "C" int mx_exec_execute_loop(mx_executable* e, mx_buffer* const* input_sets, int n_sets, int n_inputs,
                                    int iters) {
  clear_error();
  if (!e || !input_sets || n_sets < 1 || iters < 0) return set_error(MX_ERR_INVALID, "ExecuteLoop: bad arguments");
  const int n_out = (int)e->outputs.size();
  std::vector<mx_buffer*> outs(n_out);
  for (int it = 0; it < iters; ++it) {
    MX_TRY(mx_exec_execute(e, input_sets + (size_t)(it % n_sets) * n_inputs, nullptr, n_inputs, outs.data(), n_out));
    for (auto* o : outs) MX_TRY(mx_buffer_destroy(o));
  }
  return MX_OK;
}
