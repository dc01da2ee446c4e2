/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the quantized-dense path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library,
 * and only as the checker (or the timed CPU baseline), never as a product path.
 *
 * A plain-C restatement of the reference's arithmetic (github.com/gomlx/compute), compiled with
 * -ffp-contract=off so every f32 multiply/add rounds separately, as Go compiles it on amd64
 * (no FMA fusion at the default GOAMD64=v1).  Each function cites the reference code it follows.
 * How each function is pinned (golden vectors, closed forms, brute force) is listed in
 * tests/test_oracle.py.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* dtypes.DType values (dtypes/dtype_enum.go:20-140). */
enum { DT_INT8 = 2, DT_UINT8 = 6, DT_INT4 = 21, DT_UINT4 = 22 };
enum { ACT_NONE = 0, ACT_GELU = 1, ACT_RELU = 2, ACT_SILU = 3, ACT_HARDSWISH = 4, ACT_TANH = 5 };
enum { QUANT_LINEAR = 0, QUANT_NF4 = 1 };

/* unpackInt4Nibbles / unpackUint4Nibbles (internal/gobackend/ops/convertdtype.go:202-222):
 * low nibble is the first element; signed nibbles 8..15 are -8..-1 (arithmetic shift for the
 * high nibble). */
void oracle_unpack_int4(const uint8_t* packed, size_t nbytes, int8_t* dst) {
  for (size_t i = 0; i < nbytes; ++i) {
    uint8_t b = packed[i];
    int8_t lo = (int8_t)(b & 0x0F);
    if (lo >= 8) lo -= 16;
    int8_t hi = (int8_t)((int8_t)b >> 4);
    dst[2 * i] = lo;
    dst[2 * i + 1] = hi;
  }
}

void oracle_unpack_uint4(const uint8_t* packed, size_t nbytes, int8_t* dst) {
  for (size_t i = 0; i < nbytes; ++i) {
    dst[2 * i] = (int8_t)(packed[i] & 0x0F);
    dst[2 * i + 1] = (int8_t)(packed[i] >> 4);
  }
}

/* bfloat16.FromFloat32 (dtypes/bfloat16/bfloat16.go:30-39). */
uint16_t oracle_f32_to_bf16(float x) {
  uint32_t bits;
  memcpy(&bits, &x, 4);
  if ((bits & 0x7F800000u) == 0x7F800000u) return (uint16_t)(bits >> 16);
  bits += 0x7FFFu + ((bits >> 16) & 1u);
  return (uint16_t)(bits >> 16);
}

void oracle_f32_to_bf16_array(const float* x, size_t n, uint16_t* out) {
  for (size_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16(x[i]);
}

/* fusedDenseApplyActivation[float32] (internal/gobackend/fusedops/dense.go:176-205) with
 * geluChunk (gelu.go:113-118). */
float oracle_act(float x, int act) {
  switch (act) {
    case ACT_GELU: {
      const float sqrt2inv = (float)(1.0 / sqrt(2.0));
      float t = x * sqrt2inv;
      float e = (float)erf((double)t);
      float h = x * 0.5f;
      return h * (1.0f + e);
    }
    case ACT_RELU:
      return x < 0 ? 0.0f : x;
    case ACT_SILU: {
      float e = (float)exp((double)(-x));
      return x / (1.0f + e);
    }
    case ACT_HARDSWISH: {
      const float scale = (float)(1.0 / 6.0);
      float v = x * scale;
      v = v + 0.5f;
      if (v != v) return v; /* Go's min/max propagate NaN */
      v = v > 0.0f ? v : 0.0f;
      v = v < 1.0f ? v : 1.0f;
      return x * v;
    }
    case ACT_TANH:
      return (float)tanh((double)x);
    default:
      return x;
  }
}

void oracle_act_array(float* x, size_t n, int act) {
  for (size_t i = 0; i < n; ++i) x[i] = oracle_act(x[i], act);
}

/* compute.NF4LookupTable (fused_ops.go:116-121). */
static const float kNF4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

float oracle_nf4(int i) { return kNF4[i & 15]; }

static inline int weight_at(const void* w, int wdt, int64_t i) {
  switch (wdt) {
    case DT_INT8: return ((const int8_t*)w)[i];
    case DT_UINT8: return ((const uint8_t*)w)[i];
    case DT_INT4: {
      uint8_t b = ((const uint8_t*)w)[i >> 1];
      if (i & 1) return (int)((int8_t)b >> 4);
      int lo = b & 0x0F;
      return lo >= 8 ? lo - 16 : lo;
    }
    default: {
      uint8_t b = ((const uint8_t*)w)[i >> 1];
      return (i & 1) ? (b >> 4) : (b & 0x0F);
    }
  }
}

/*
 * quantizedDenseLinearInt / quantizedDenseNF4 (internal/gobackend/fusedops/quantizeddense.go:
 * 586-650), then the activation (:416).  Computes rows [m_begin, m_end) of the output:
 *   out[m,n] = bias[n] (or 0); for k = 0..K-1 in order:
 *     Linear:            out += (x[m,k] * float32(w[k,n])) * s
 *     Linear + zp:       out += x[m,k] * (float32(w[k,n]) * s + zp)
 *     NF4:               out += (x[m,k] * NF4[uint8(w[k,n]) & 15]) * s
 *   with s = scale[k, n/B] for block_axis 1 (the reference layout) or scale[k/B, n] for
 *   block_axis 0 (blocks along K: the per-element value of the reference-executable form whose
 *   scale is expanded to [K, N] with BlockSize 1).
 * x, scale, zp, bias are f32 (bf16 inputs are widened exactly by the caller).  Output f32.
 * `threads` > 1 splits the work like quantizedDenseParallel (:528-579): rows when M > 1, column
 * tiles when M == 1; each output element is computed by one thread in the same order, so the
 * result does not depend on the thread count.
 */
void oracle_qdense(const float* x, const void* w, int wdt, const float* scale, const float* zp,
                   const float* bias, float* out, int64_t M, int64_t K, int64_t N, int scheme,
                   int block_axis, int64_t B, int act, int64_t m_begin, int64_t m_end, int threads) {
  const int64_t nb = (N + B - 1) / B;
  const int64_t rows = m_end - m_begin;
  const int64_t tile = M == 1 ? (4096 / (K > 0 ? K : 1) > 1 ? 4096 / (K > 0 ? K : 1) : 1) : N;
  const int64_t ntiles = (N + tile - 1) / tile;
  const int64_t units = rows * ntiles;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
#endif
  for (int64_t u = 0; u < units; ++u) {
    const int64_t m = m_begin + u / ntiles;
    const int64_t n0 = (u % ntiles) * tile;
    const int64_t n1 = n0 + tile < N ? n0 + tile : N;
    float* o = out + (m - m_begin) * N;
    for (int64_t n = n0; n < n1; ++n) o[n] = bias ? bias[n] : 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float xv = x[(m - m_begin) * K + k];
      for (int64_t n = n0; n < n1; ++n) {
        const int64_t si = block_axis == 1 ? k * nb + n / B : (k / B) * N + n;
        const int wi = weight_at(w, wdt, k * N + n);
        const float s = scale[si];
        if (scheme == QUANT_NF4) {
          float t = xv * kNF4[(uint8_t)wi & 0x0F];
          t = t * s;
          o[n] = o[n] + t;
        } else if (zp) {
          float u2 = (float)wi * s;
          u2 = u2 + zp[si];
          float t = xv * u2;
          o[n] = o[n] + t;
        } else {
          float t = xv * (float)wi;
          t = t * s;
          o[n] = o[n] + t;
        }
      }
    }
    for (int64_t n = n0; n < n1; ++n) o[n] = oracle_act(o[n], act);
  }
  (void)threads;
}

/* Same computation in f64 (no rounding inside the sum): the "mathematical" value used to bound
 * the f32 accumulation error of the fast GPU kernels. */
void oracle_qdense_f64(const float* x, const void* w, int wdt, const float* scale, const float* zp,
                       const float* bias, double* out, int64_t M, int64_t K, int64_t N, int scheme,
                       int block_axis, int64_t B, int64_t m_begin, int64_t m_end) {
  const int64_t nb = (N + B - 1) / B;
  (void)M;
  for (int64_t m = m_begin; m < m_end; ++m) {
    double* o = out + (m - m_begin) * N;
    for (int64_t n = 0; n < N; ++n) o[n] = bias ? bias[n] : 0.0;
    for (int64_t k = 0; k < K; ++k) {
      const double xv = x[(m - m_begin) * K + k];
      for (int64_t n = 0; n < N; ++n) {
        const int64_t si = block_axis == 1 ? k * nb + n / B : (k / B) * N + n;
        const int wi = weight_at(w, wdt, k * N + n);
        const double wf = scheme == QUANT_NF4 ? (double)kNF4[(uint8_t)wi & 0x0F] : (double)wi;
        const double u = zp ? wf * scale[si] + zp[si] : wf * scale[si];
        o[n] += xv * u;
      }
    }
  }
}

/* Sum of |terms| per output: the scale of the rounding error of any summation order. */
void oracle_qdense_abs(const float* x, const void* w, int wdt, const float* scale, const float* zp,
                       const float* bias, double* out, int64_t M, int64_t K, int64_t N, int scheme,
                       int block_axis, int64_t B, int64_t m_begin, int64_t m_end) {
  const int64_t nb = (N + B - 1) / B;
  (void)M;
  for (int64_t m = m_begin; m < m_end; ++m) {
    double* o = out + (m - m_begin) * N;
    for (int64_t n = 0; n < N; ++n) o[n] = bias ? fabs((double)bias[n]) : 0.0;
    for (int64_t k = 0; k < K; ++k) {
      const double xv = fabs((double)x[(m - m_begin) * K + k]);
      for (int64_t n = 0; n < N; ++n) {
        const int64_t si = block_axis == 1 ? k * nb + n / B : (k / B) * N + n;
        const int wi = weight_at(w, wdt, k * N + n);
        const double wf = scheme == QUANT_NF4 ? (double)kNF4[(uint8_t)wi & 0x0F] : (double)wi;
        const double u = zp ? wf * scale[si] + zp[si] : wf * scale[si];
        o[n] += xv * fabs(u);
      }
    }
  }
}
