// Device helpers shared by the HIP kernels: bf16 conversion, scalar loads by dtype, weight
// decoding and the activation epilogue with the reference's exact arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mxrt.h"

namespace mx {

// ---------------------------------------------------------------------------------------------
// Single-rounded f32 arithmetic that is never contracted into an FMA.  HIP's __fadd_rn and
// __fmul_rn are plain `+`/`*` here (no OCML rounded operations), which clang fuses into FMAs
// under its default -ffp-contract for HIP; the reference's Go loops round every product and sum
// separately, so reference-order code uses these instead.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float div_rn(float a, float b) {
#pragma clang fp contract(off)
  return a / b;
}

// ---------------------------------------------------------------------------------------------
// bf16 <-> f32.  f32 -> bf16 follows bfloat16.FromFloat32 (dtypes/bfloat16/bfloat16.go:30-39):
// NaN/Inf keep their top 16 bits, everything else rounds to nearest even.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t bits = __float_as_uint(f);
  if ((bits & 0x7F800000u) == 0x7F800000u) return (uint16_t)(bits >> 16);
  bits += 0x7FFFu + ((bits >> 16) & 1u);
  return (uint16_t)(bits >> 16);
}

// IEEE half (fp16) <-> f32 via the hardware conversion (round to nearest even).
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  _Float16 v = (_Float16)f;
  return __builtin_bit_cast(uint16_t, v);
}

// Loads element i of a float32 / bfloat16 array as f32.
__device__ __forceinline__ float load_f(const void* p, int64_t i, int dt) {
  if (dt == MX_DTYPE_BFLOAT16) return bf16_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

__device__ __forceinline__ void store_f(void* p, int64_t i, int dt, float v) {
  if (dt == MX_DTYPE_BFLOAT16)
    ((uint16_t*)p)[i] = f32_to_bf16(v);
  else
    ((float*)p)[i] = v;
}

// ---------------------------------------------------------------------------------------------
// Weight decoding.  Packed 4-bit storage follows the reference packing: flat element i lives in
// byte i/2, low nibble when i is even (internal/gobackend/ops/convertdtype.go:202-222); signed
// nibbles 8..15 mean -8..-1.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ int decode_weight(const void* w, int64_t i, int wdt) {
  switch (wdt) {
    case MX_DTYPE_INT8: return (int)((const int8_t*)w)[i];
    case MX_DTYPE_UINT8: return (int)((const uint8_t*)w)[i];
    case MX_DTYPE_INT4: {
      uint32_t b = ((const uint8_t*)w)[i >> 1];
      int nib = (i & 1) ? (int)(b >> 4) : (int)(b & 15u);
      return nib >= 8 ? nib - 16 : nib;
    }
    default: {  // MX_DTYPE_UINT4
      uint32_t b = ((const uint8_t*)w)[i >> 1];
      return (i & 1) ? (int)(b >> 4) : (int)(b & 15u);
    }
  }
}

// QLoRA NormalFloat4 table (fused_ops.go:116-121).
__constant__ static const float kNF4Table[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

// ---------------------------------------------------------------------------------------------
// Activation epilogue with the reference's arithmetic (fusedops/dense.go:176-205 and
// gelu.go:113-118): f32 values, transcendental parts evaluated in f64 and rounded to f32, and
// no contraction of separate multiply/add steps.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float act_ref(float x, int act) {
  switch (act) {
    case MX_ACT_GELU: {
      // x * 0.5 * (1 + float32(erf(float64(x * float32(1/sqrt(2))))))
      float t = mul_rn(x, __uint_as_float(0x3f3504f3u));
      float e = (float)erf((double)t);
      return mul_rn(mul_rn(x, 0.5f), add_rn(1.0f, e));
    }
    case MX_ACT_RELU:
      return x < 0.0f ? 0.0f : x;
    case MX_ACT_SILU: {
      float e = (float)exp((double)(-x));
      return div_rn(x, add_rn(1.0f, e));
    }
    case MX_ACT_HARDSWISH: {
      // shapeX := min(max(x*float32(1/6) + 0.5, 0), 1); x * shapeX  (Go min/max propagate NaN)
      float v = add_rn(mul_rn(x, __uint_as_float(0x3e2aaaabu)), 0.5f);
      if (v != v) return v;
      v = v > 0.0f ? v : 0.0f;
      v = v < 1.0f ? v : 1.0f;
      return mul_rn(x, v);
    }
    case MX_ACT_TANH:
      return (float)tanh((double)x);
    default:
      return x;
  }
}

// erf(x) by the rational-exponential approximation of Abramowitz & Stegun, Handbook of
// Mathematical Functions, 7.1.26 (|error| <= 1.5e-7): one reciprocal, one exp, six FMAs and no
// branches.  The reference rounds erf to f32 before adding 1 (an absolute step of 6e-8 near -1),
// so the two agree to a few of those steps.
__device__ __forceinline__ float erf_as7126(float x) {
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, ax, 1.0f));
  float p = fmaf(1.061405429f, t, -1.453152027f);
  p = fmaf(p, t, 1.421413741f);
  p = fmaf(p, t, -0.284496736f);
  p = fmaf(p, t, 0.254829592f);
  const float r = fmaf(-p * t, __expf(-ax * ax), 1.0f);
  return copysignf(r, x);
}

// Activation epilogue of the fast kernels, in f32 (erf_as7126, hardware exp and reciprocal, OCML
// tanhf): absolute differences from act_ref of order 1e-7, far below the bf16 rounding of their
// outputs.
__device__ __forceinline__ float act_fast(float x, int act) {
  switch (act) {
    case MX_ACT_GELU:
      return 0.5f * x * (1.0f + erf_as7126(x * 0.70710678118654752f));
    case MX_ACT_RELU:
      return x < 0.0f ? 0.0f : x;
    case MX_ACT_SILU:
      return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
    case MX_ACT_HARDSWISH: {
      float v = x * (1.0f / 6.0f) + 0.5f;
      if (v != v) return v;
      v = v > 0.0f ? v : 0.0f;
      v = v < 1.0f ? v : 1.0f;
      return x * v;
    }
    case MX_ACT_TANH:
      return tanhf(x);
    default:
      return x;
  }
}

}  // namespace mx
