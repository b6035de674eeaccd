/*
 * oct_oracle_fft.c -- CPU restatement of Oct's binary64 FFT contract.
 *
 * TEST INFRASTRUCTURE ONLY (see oct_oracle.c).  Restates
 * internal/fft/fft.go:218-258: roots() builds n/2 twiddles
 * w_j = cos(a) + i sin(a) with a = -2*pi/n * j, and cpuWithRoots() performs an
 * in-place bit-reversal permutation followed by iterative radix-2
 * decimation-in-time butterflies t = w[j*(n/span)] * x[b+j+half],
 * x[b+j] = a + t, x[b+j+half] = a - t (forward, unnormalised).  The complex
 * product is Go's (xu - yv) + (xv + yu)i with every product and sum rounded
 * (compiled with -ffp-contract=off, as Go's amd64 code at GOAMD64=v1).
 *
 * Pinned in tests/test_oracle_fft.py by the Oct FFT facts
 * (Language/Prometheus/gpu/fft.octest:7-28, valid/fft_contract.octest:3-11),
 * closed forms (impulse, constant, single tone), an O(n^2) DFT in extended
 * precision, numpy.fft (an independent library), linearity and Parseval.
 */
#include <math.h>
#include <stdint.h>

#include "oct_oracle.h"

void oct_fft64_roots(double* twiddles, uint32_t n) {
  const double pi = 3.14159265358979323846;
  for (uint32_t j = 0; j < n / 2; ++j) {
    const double angle = -2.0 * pi / (double)n * (double)j;
    twiddles[2 * j] = cos(angle);
    twiddles[2 * j + 1] = sin(angle);
  }
}

void oct_fft64_with_roots(const double* input, double* output, const double* twiddles, uint32_t n) {
  for (uint32_t i = 0; i < 2 * n; ++i) output[i] = input[i];
  for (uint32_t i = 1, j = 0; i < n; ++i) {
    uint32_t bit = n >> 1;
    for (; j & bit; bit >>= 1) j ^= bit;
    j ^= bit;
    if (i < j) {
      const double re = output[2 * i], im = output[2 * i + 1];
      output[2 * i] = output[2 * j];
      output[2 * i + 1] = output[2 * j + 1];
      output[2 * j] = re;
      output[2 * j + 1] = im;
    }
  }
  for (uint32_t span = 2; span <= n; span *= 2) {
    const uint32_t half = span / 2;
    for (uint32_t base = 0; base < n; base += span) {
      for (uint32_t j = 0; j < half; ++j) {
        const double wr = twiddles[2 * (j * (n / span))], wi = twiddles[2 * (j * (n / span)) + 1];
        const uint32_t p = base + j, q = base + j + half;
        const double vr = output[2 * q], vi = output[2 * q + 1];
        const double tr = wr * vr - wi * vi;
        const double ti = wr * vi + wi * vr;
        const double ar = output[2 * p], ai = output[2 * p + 1];
        output[2 * p] = ar + tr;
        output[2 * p + 1] = ai + ti;
        output[2 * q] = ar - tr;
        output[2 * q + 1] = ai - ti;
      }
    }
  }
}

int32_t oct_fft64(const double* input, double* output, double* scratch_twiddles, uint32_t n) {
  if (input == 0 || output == 0 || n == 0 || (n & (n - 1)) != 0) return 1;
  if (n > 1) oct_fft64_roots(scratch_twiddles, n);
  oct_fft64_with_roots(input, output, scratch_twiddles, n);
  return 0;
}

/* internal/fft/fft.go:176-192 (agrees): every component within
   1e-12 * max|component of reference| + n * 4.9e-324, all finite.
   Returns 1 when they agree, 0 otherwise. */
int32_t oct_fft64_agrees(const double* reference, const double* actual, uint32_t n) {
  double scale = 0.0;
  for (uint32_t i = 0; i < 2 * n; ++i) scale = fmax(scale, fabs(reference[i]));
  const double tolerance = 1e-12 * scale + 4.9406564584124654e-324 * (double)n;
  for (uint32_t i = 0; i < 2 * n; ++i) {
    if (!isfinite(actual[i]) || !isfinite(reference[i])) return 0;
    if (fabs(actual[i] - reference[i]) > tolerance) return 0;
  }
  return 1;
}

/*
 * The batched complex-fp32 FFT's acceptance authority
 * (internal/prometheus/native/Marionette/reactor_fft_api_tests.cpp:525-553):
 * for each batch b (base b * stride) a direct binary64 DFT
 * X[k] = sum_s x[s] * (cos a + i sin a), a = -+2*pi*(k*s)/n (k*s a 32-bit
 * product, as there), divided by n for the inverse, rounded to fp32.  The
 * padding between batches is copied from the input.  O(n^2) per batch.
 */
void oct_dft_c32(const float* input, float* output, uint32_t n, uint32_t batch, uint32_t stride, int32_t inverse) {
  const double pi = 3.14159265358979323846264338327950288;
  const uint64_t physical = (uint64_t)(batch - 1u) * stride + n;
  for (uint64_t i = 0; i < 2 * physical; ++i) output[i] = input[i];
  for (uint32_t b = 0; b < batch; ++b) {
    const uint64_t base = (uint64_t)b * stride;
    for (uint32_t k = 0; k < n; ++k) {
      double re = 0.0, im = 0.0;
      for (uint32_t s = 0; s < n; ++s) {
        const double angle = (inverse ? 2.0 : -2.0) * pi * (double)(uint32_t)(k * s) / (double)n;
        const double c = cos(angle), sn = sin(angle);
        const double xr = input[2 * (base + s)], xi = input[2 * (base + s) + 1];
        re += xr * c - xi * sn;
        im += xr * sn + xi * c;
      }
      if (inverse) {
        re /= (double)n;
        im /= (double)n;
      }
      output[2 * (base + k)] = (float)re;
      output[2 * (base + k) + 1] = (float)im;
    }
  }
}
