/*
 * oracle/q4_0_ref.c - TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of the reference's GGUF Q4_0 handling, used as the
 * checker for the HIP kernels.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product never does.
 *
 *  - block decode: src/spark_vllm_ascend/integration/weights.py:34-40
 *    (d = fp16 LE bytes 0-1; element j<16 = (qs[j] & 15) - 8,
 *     j>=16 = (qs[j-16] >> 4) - 8)
 *  - dequantise to fp32 (exact: an 11-bit significand times a 4-bit
 *    integer) then to bf16 with round-to-nearest-even:
 *    src/spark_vllm_ascend/integration/weights.py:28-32,
 *    src/tools/deployment/prepare_model.py:62-64
 *  - GEMV numerics: src/spark_vllm_ascend/kernels/linear.py:16-200
 *    (fp32 accumulation of x times the bf16 weight, bf16 output)
 *
 * fp16 decoding is written from the IEEE 754 binary16 definition with
 * ldexp, independently of numpy's float16, so the two restatements can
 * check each other.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float f16_to_f32(uint16_t h) {
  const int sign = (h >> 15) & 1;
  const int e = (h >> 10) & 0x1f;
  const int m = h & 0x3ff;
  float v;
  if (e == 0)
    v = ldexpf((float)m, -24); /* zero or subnormal: m * 2^-24 */
  else if (e == 31)
    v = m ? NAN : INFINITY;
  else
    v = ldexpf((float)(m | 0x400), e - 25); /* (1024 + m) * 2^(e - 15 - 10) */
  return sign ? -v : v;
}

static uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float bf16_to_f32(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float oracle_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t oracle_f32_to_bf16(float f) { return f32_to_bf16_rne(f); }

/* codes: [n, k] int8 in [-8, 7]; scales: [n, k/32] fp16 bits */
void oracle_q4_0_unpack(const uint8_t* blocks, int64_t n, int64_t k, int8_t* codes,
                        uint16_t* scales) {
  const int64_t nb = k / 32;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t* blk = blocks + (r * nb + b) * 18;
      scales[r * nb + b] = (uint16_t)(blk[0] | (blk[1] << 8));
      int8_t* c = codes + r * k + b * 32;
      for (int j = 0; j < 16; ++j) {
        c[j] = (int8_t)((blk[2 + j] & 15) - 8);
        c[16 + j] = (int8_t)((blk[2 + j] >> 4) - 8);
      }
    }
}

void oracle_q4_0_dequant_f32(const uint8_t* blocks, int64_t n, int64_t k, float* out) {
  const int64_t nb = k / 32;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t* blk = blocks + (r * nb + b) * 18;
      const float d = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
      float* o = out + r * k + b * 32;
      for (int j = 0; j < 16; ++j) {
        o[j] = d * (float)((blk[2 + j] & 15) - 8);
        o[16 + j] = d * (float)((blk[2 + j] >> 4) - 8);
      }
    }
}

void oracle_q4_0_dequant_bf16(const uint8_t* blocks, int64_t n, int64_t k, uint16_t* out) {
  const int64_t nb = k / 32;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t* blk = blocks + (r * nb + b) * 18;
      const float d = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
      uint16_t* o = out + r * k + b * 32;
      for (int j = 0; j < 16; ++j) {
        o[j] = f32_to_bf16_rne(d * (float)((blk[2 + j] & 15) - 8));
        o[16 + j] = f32_to_bf16_rne(d * (float)((blk[2 + j] >> 4) - 8));
      }
    }
}

/* y[r] = sum_j x_j * w_rj in double over the exactly dequantised weights. */
void oracle_q4_0_gemv_f64(const uint16_t* x, const uint8_t* blocks, int64_t n, int64_t k,
                          double* y) {
  const int64_t nb = k / 32;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n; ++r) {
    double acc = 0.0;
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t* blk = blocks + (r * nb + b) * 18;
      const double d = (double)f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
      const uint16_t* xb = x + b * 32;
      for (int j = 0; j < 16; ++j) {
        acc += (double)bf16_to_f32(xb[j]) * d * (double)((blk[2 + j] & 15) - 8);
        acc += (double)bf16_to_f32(xb[16 + j]) * d * (double)((blk[2 + j] >> 4) - 8);
      }
    }
    y[r] = acc;
  }
}

/* The reference device kernel's rounding points: weight = bf16(d * q),
 * fp32 multiply-add with the fp32 activation, bf16 output (sequential
 * accumulation order; the reference's lane order is not reproduced). */
void oracle_q4_0_gemv_bf16w(const uint16_t* x, const uint8_t* blocks, int64_t n, int64_t k,
                            uint16_t* y) {
  const int64_t nb = k / 32;
  for (int64_t r = 0; r < n; ++r) {
    float acc = 0.f;
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t* blk = blocks + (r * nb + b) * 18;
      const float d = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
      const uint16_t* xb = x + b * 32;
      for (int j = 0; j < 16; ++j) {
        const float wl = bf16_to_f32(f32_to_bf16_rne(d * (float)((blk[2 + j] & 15) - 8)));
        const float wh = bf16_to_f32(f32_to_bf16_rne(d * (float)((blk[2 + j] >> 4) - 8)));
        acc = fmaf(bf16_to_f32(xb[j]), wl, acc);
        acc = fmaf(bf16_to_f32(xb[16 + j]), wh, acc);
      }
    }
    y[r] = f32_to_bf16_rne(acc);
  }
}
