/*
 * oct_oracle_m1.c -- CPU restatement of the Gemma-4-E2B M1 stages.
 *
 * TEST INFRASTRUCTURE ONLY (see oct_oracle.c).  Restates:
 *   oct_m1_rmsnorm       the reference's independent double-sum RMSNorm oracle
 *                        (native/Marionette/reactor_concept_rmsnorm_tests.cpp:17-36):
 *                        x optionally BF16-rounded, sum(x^2) in binary64,
 *                        inv = (float)(1/sqrt(sum/W + eps)), y = x*inv*w,
 *                        y optionally BF16-rounded;
 *   oct_m1_head_rmsnorm_go  the Go witness cpuHeadRMSNorm
 *                        (internal/prometheus/gemma4e2b_m1_rtx.go:811-832):
 *                        float sum, inv = float32(1/math.Sqrt(float64(sum/W + eps)));
 *   oct_m1_rope          cpuGemma4e2bRope (gemma4e2b_m1_rtx.go:834-861) and
 *                        shaders/.../gemma4e2b/rope_half_split.sdslv: BF16 of
 *                        each product and of the difference / sum;
 *   oct_m1_raw_scores    cpuGemma4e2bRawScores (gemma4e2b_m1_rtx.go:863-883):
 *                        float accumulation in channel order, times 0.0625.
 * Pinned in tests/test_oracle_m1.py.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "oct_oracle.h"

static float bf16r(float v) { return oct_bf16_to_f32(oct_f32_to_bf16(v)); }

void oct_m1_rmsnorm(const float* input, uint32_t stride, const float* weight, float* output, float* inv_rms,
                    uint32_t rows, uint32_t width, float epsilon, int32_t round_in, int32_t round_out) {
  for (uint32_t r = 0; r < rows; ++r) {
    double sum = 0.0;
    for (uint32_t c = 0; c < width; ++c) {
      const double x = round_in ? bf16r(input[(size_t)r * stride + c]) : input[(size_t)r * stride + c];
      sum += x * x;
    }
    const float inv = (float)(1.0 / sqrt(sum / width + epsilon));
    if (inv_rms) inv_rms[r] = inv;
    for (uint32_t c = 0; c < width; ++c) {
      const float x = round_in ? bf16r(input[(size_t)r * stride + c]) : input[(size_t)r * stride + c];
      const float v = x * inv * weight[c];
      output[(size_t)r * width + c] = round_out ? bf16r(v) : v;
    }
  }
}

void oct_m1_head_rmsnorm_go(const float* input, const float* weight, float* output, uint32_t rows, uint32_t width,
                            float epsilon) {
  for (uint32_t r = 0; r < rows; ++r) {
    float sum = 0.0f;
    for (uint32_t c = 0; c < width; ++c) {
      const float v = input[(size_t)r * width + c];
      sum += v * v;
    }
    const float inv = (float)(1.0 / sqrt((double)(sum / (float)width + epsilon)));
    for (uint32_t c = 0; c < width; ++c)
      output[(size_t)r * width + c] = input[(size_t)r * width + c] * inv * weight[c];
  }
}

void oct_m1_rope(const float* source, const float* cosine, const float* sine, float* output, uint32_t tokens,
                 uint32_t heads, uint32_t width) {
  const uint32_t half = width / 2;
  for (uint32_t t = 0; t < tokens; ++t)
    for (uint32_t h = 0; h < heads; ++h) {
      const size_t base = ((size_t)t * heads + h) * width;
      for (uint32_t c = 0; c < width; ++c) {
        const uint32_t f = c % half;
        const size_t mate = c >= half ? base + f : base + f + half;
        const float first = bf16r(source[base + c] * cosine[(size_t)t * width + f]);
        const float second = bf16r(source[mate] * sine[(size_t)t * width + f]);
        output[base + c] = bf16r(c >= half ? first + second : first - second);
      }
    }
}

void oct_m1_raw_scores(const float* query, const float* key, float* scores, uint32_t tokens, uint32_t query_heads,
                       uint32_t width, float scale) {
  for (uint32_t h = 0; h < query_heads; ++h)
    for (uint32_t i = 0; i < tokens; ++i)
      for (uint32_t j = 0; j < tokens; ++j) {
        const float* q = query + ((size_t)i * query_heads + h) * width;
        const float* k = key + (size_t)j * width;
        float acc = 0.0f;
        for (uint32_t c = 0; c < width; ++c) acc += q[c] * k[c];
        scores[((size_t)h * tokens + i) * tokens + j] = acc * scale;
      }
}
