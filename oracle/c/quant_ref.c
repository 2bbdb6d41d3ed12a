/* Scalar C restatement of MLX's affine quantizer (mx.quantize, CPU semantics), used to
 * cross-check the numpy restatement in oracle/quantize.py. TEST INFRASTRUCTURE ONLY.
 * Per group: fp32 min/max, s = max((max-min)/n, 1e-7) (negated unless |min| > |max|),
 * edge trick q0 = rint(edge/s), codes = clamp(rint((x-b)/s), 0, n). Built with
 * -ffp-contract=off so every step is one IEEE fp32 operation. */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

void kvq_ref_quantize(const float* x, size_t rows, int D, int G, int bits, uint32_t* codes, float* scales,
                      float* biases) {
  const float n_bins = (float)((1 << bits) - 1);
  const float eps = 1e-7f;
  const int per = 32 / bits;
  for (size_t r = 0; r < rows; ++r) {
    const float* xr = x + r * (size_t)D;
    uint32_t* cr = codes + r * (size_t)(D / per);
    for (int g = 0; g < D / G; ++g) {
      const float* xg = xr + g * G;
      float w_max = -INFINITY, w_min = INFINITY;
      for (int j = 0; j < G; ++j) {
        w_max = xg[j] > w_max ? xg[j] : w_max;
        w_min = xg[j] < w_min ? xg[j] : w_min;
      }
      const int mask = fabsf(w_min) > fabsf(w_max);
      float scale = (w_max - w_min) / n_bins;
      scale = scale > eps ? scale : eps;
      scale = mask ? scale : -scale;
      const float edge = mask ? w_min : w_max;
      const float q0 = rintf(edge / scale);
      float bias = 0.0f;
      if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
      }
      for (int j = 0; j < G; ++j) {
        float c = rintf((xg[j] - bias) / scale);
        c = c < 0.0f ? 0.0f : (c > n_bins ? n_bins : c);
        const int d = g * G + j;
        if (d % per == 0) cr[d / per] = 0;
        cr[d / per] |= ((uint32_t)c) << ((d % per) * bits);
      }
      scales[r * (size_t)(D / G) + g] = scale;
      biases[r * (size_t)(D / G) + g] = bias;
    }
  }
}
