/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the GGML block-format paths.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library,
 * and only as the checker, never as a product path.
 *
 * A plain-C restatement of the reference's GGML dequantisation, fused dense product and
 * quantized embedding lookup (github.com/gomlx/compute), compiled with -ffp-contract=off so
 * every f32 multiply/add rounds separately, as Go compiles it on amd64.  Each function cites the
 * reference code it follows.  How each one is pinned (closed forms, independent encoders, library
 * conversions, brute force) is listed in tests/test_oracle_ggml.py.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* compute.GGMLQuantType values (fused_ops.go:134-146). */
enum { GGML_Q4_0 = 0, GGML_Q8_0 = 1, GGML_IQ4_NL = 2, GGML_Q4_K = 5, GGML_Q6_K = 7 };

float oracle_act(float x, int act); /* qdense_ref.c */

/* Float16.Float32 (dtypes/float16/float16.go:17-60): exact IEEE half -> single, NaN payload
 * shifted into the top of the single mantissa. */
float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  int exp = (h & 0x7C00u) >> 10;
  uint32_t mant = h & 0x03FFu;
  uint32_t bits;
  if (exp == 0x1F) {
    bits = sign | 0x7F800000u | (mant << 13);
  } else if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      /* Subnormal: shift the leading one into bit 10, adjusting the exponent. */
      int e = 1;
      while ((mant & 0x0400u) == 0) {
        mant <<= 1;
        --e;
      }
      mant &= 0x03FFu;
      bits = sign | ((uint32_t)(e - 15 + 127) << 23) | (mant << 13);
    }
  } else {
    bits = sign | ((uint32_t)(exp - 15 + 127) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* The same over an array, writing the f32 bit patterns (no float round trip that would quiet a
 * signalling NaN). */
void oracle_f16_to_f32_array(const uint16_t* h, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) {
    const float f = oracle_f16_to_f32(h[i]);
    memcpy(out + i, &f, 4);
  }
}

/* ggmlFp16LE (quantizeddense_ggml.go:153-156). */
static float fp16le(const uint8_t* p) { return oracle_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* compute.IQ4NLLookupTable (fused_ops.go:127-130). */
static const float kIQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

int oracle_ggml_values_per_block(int type) {
  switch (type) {
    case GGML_Q4_0: case GGML_Q8_0: case GGML_IQ4_NL: return 32;
    case GGML_Q4_K: case GGML_Q6_K: return 256;
    default: return 0;
  }
}

int oracle_ggml_bytes_per_block(int type) {
  switch (type) {
    case GGML_Q4_0: case GGML_IQ4_NL: return 18;
    case GGML_Q8_0: return 34;
    case GGML_Q4_K: return 144;
    case GGML_Q6_K: return 210;
    default: return 0;
  }
}

/* getScaleMinK4 (quantizeddense_ggml.go:229-239). */
static void scale_min_k4(int j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
    *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
}

/* One row of blocks -> K f32 values: dequantQ8_0Row / dequantQ4_0Row / dequantIQ4NLRow /
 * dequantQ4_KRow / dequantQ6_KRow (quantizeddense_ggml.go:158-302).  Returns -1 for an
 * unsupported type. */
int oracle_ggml_dequant_row(int type, const uint8_t* row, int64_t bytes_per_row, float* out) {
  const int bpb = oracle_ggml_bytes_per_block(type);
  if (bpb == 0) return -1;
  const int64_t nb = bytes_per_row / bpb;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* blk = row + b * bpb;
    switch (type) {
      case GGML_Q8_0: {
        const float d = fp16le(blk);
        float* o = out + b * 32;
        for (int i = 0; i < 32; ++i) o[i] = d * (float)(int8_t)blk[2 + i];
        break;
      }
      case GGML_Q4_0: {
        const float d = fp16le(blk);
        float* o = out + b * 32;
        for (int i = 0; i < 16; ++i) {
          o[i] = d * (float)((int)(blk[2 + i] & 0x0F) - 8);
          o[16 + i] = d * (float)((int)(blk[2 + i] >> 4) - 8);
        }
        break;
      }
      case GGML_IQ4_NL: {
        const float d = fp16le(blk);
        float* o = out + b * 32;
        for (int i = 0; i < 16; ++i) {
          o[i] = d * kIQ4NL[blk[2 + i] & 0x0F];
          o[16 + i] = d * kIQ4NL[blk[2 + i] >> 4];
        }
        break;
      }
      case GGML_Q4_K: {
        const float d = fp16le(blk), dmin = fp16le(blk + 2);
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        float* o = out + b * 256;
        int idx = 0;
        for (int chunk = 0; chunk < 4; ++chunk) {
          uint8_t sc1, m1, sc2, m2;
          scale_min_k4(2 * chunk, scales, &sc1, &m1);
          scale_min_k4(2 * chunk + 1, scales, &sc2, &m2);
          const float d1 = d * (float)sc1, min1 = dmin * (float)m1;
          const float d2 = d * (float)sc2, min2 = dmin * (float)m2;
          const uint8_t* q = qs + 32 * chunk;
          for (int l = 0; l < 32; ++l) o[idx++] = d1 * (float)(q[l] & 0xF) - min1;
          for (int l = 0; l < 32; ++l) o[idx++] = d2 * (float)(q[l] >> 4) - min2;
        }
        break;
      }
      case GGML_Q6_K: {
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const uint8_t* sc = blk + 192;
        const float d = fp16le(blk + 208);
        float* o = out + b * 256;
        for (int half = 0; half < 2; ++half) {
          const uint8_t* l0 = ql + 64 * half;
          const uint8_t* h0 = qh + 32 * half;
          const uint8_t* s0 = sc + 8 * half;
          float* oh = o + 128 * half;
          for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = (int8_t)((l0[l] & 0xF) | ((h0[l] & 3) << 4)) - 32;
            const int q2 = (int8_t)((l0[l + 32] & 0xF) | (((h0[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int8_t)((l0[l] >> 4) | (((h0[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int8_t)((l0[l + 32] >> 4) | (((h0[l] >> 6) & 3) << 4)) - 32;
            oh[l] = d * (float)(int8_t)s0[is] * (float)q1;
            oh[l + 32] = d * (float)(int8_t)s0[is + 2] * (float)q2;
            oh[l + 64] = d * (float)(int8_t)s0[is + 4] * (float)q3;
            oh[l + 96] = d * (float)(int8_t)s0[is + 6] * (float)q4;
          }
        }
        break;
      }
      default:
        return -1;
    }
  }
  return 0;
}

/* quantizedDenseGGML (quantizeddense_ggml.go:103-130) then the activation epilogue
 * (dense.go:176-205): per output, the dequantised row dotted with x in k order, then the bias
 * added, then the activation (the per-worker scratch row of the reference is a per-thread buffer). */
int oracle_ggml_dense(const float* x, const uint8_t* w, int type, const float* bias, float* out, int64_t M,
                      int64_t K, int64_t N, int64_t bytes_per_row, int act) {
  const int vpb = oracle_ggml_values_per_block(type), bpb = oracle_ggml_bytes_per_block(type);
  if (vpb == 0 || bytes_per_row % bpb != 0 || (bytes_per_row / bpb) * vpb != K) return -1;
  int bad = 0;
#pragma omp parallel
  {
    float* row = (float*)malloc((size_t)(K > 0 ? K : 1) * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      if (!row) {
        bad = 1;
        continue;
      }
      oracle_ggml_dequant_row(type, w + n * bytes_per_row, bytes_per_row, row);
      for (int64_t m = 0; m < M; ++m) {
        const float* xr = x + m * K;
        float dot = 0.0f;
        for (int64_t k = 0; k < K; ++k) dot += xr[k] * row[k];
        float v = dot;
        if (bias) v += bias[n];
        out[m * N + n] = oracle_act(v, act);
      }
    }
    free(row);
  }
  return bad ? -2 : 0;
}

/* The same product in f64 with the sum of |terms| (the accumulation bound of the fast kernels);
 * the weights are the oracle's exact f32 dequantised values. */
int oracle_ggml_dense_f64(const float* x, const uint8_t* w, int type, const float* bias, double* out, double* abs_out,
                          int64_t M, int64_t K, int64_t N, int64_t bytes_per_row) {
  const int vpb = oracle_ggml_values_per_block(type), bpb = oracle_ggml_bytes_per_block(type);
  if (vpb == 0 || bytes_per_row % bpb != 0 || (bytes_per_row / bpb) * vpb != K) return -1;
#pragma omp parallel
  {
    float* row = (float*)malloc((size_t)(K > 0 ? K : 1) * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      if (!row) continue;
      oracle_ggml_dequant_row(type, w + n * bytes_per_row, bytes_per_row, row);
      for (int64_t m = 0; m < M; ++m) {
        double s = bias ? (double)bias[n] : 0.0, a = bias ? fabs((double)bias[n]) : 0.0;
        for (int64_t k = 0; k < K; ++k) {
          const double t = (double)x[m * K + k] * (double)row[k];
          s += t;
          a += fabs(t);
        }
        out[m * N + n] = s;
        abs_out[m * N + n] = a;
      }
    }
    free(row);
  }
  return 0;
}

/* execQuantizedEmbeddingLookup (quantizeddense.go:455-499): out[i] = dequant(data[idx[i]]);
 * returns the position of the first index outside [0, vocab) + 1, or 0. */
int64_t oracle_ggml_embedding(const uint8_t* data, int64_t vocab, int64_t bytes_per_row, int type,
                              const int64_t* idx, int64_t n, float* out) {
  const int vpb = oracle_ggml_values_per_block(type), bpb = oracle_ggml_bytes_per_block(type);
  if (vpb == 0 || bytes_per_row % bpb != 0) return -1;
  const int64_t K = (bytes_per_row / bpb) * vpb;
  for (int64_t i = 0; i < n; ++i) {
    if (idx[i] < 0 || idx[i] >= vocab) return i + 1;
    oracle_ggml_dequant_row(type, data + idx[i] * bytes_per_row, bytes_per_row, out + i * K);
  }
  return 0;
}
