/* FP64 CPU restatement of the reference kernels on the hot path.
 *
 * TEST INFRASTRUCTURE ONLY: this library is the checker of the gfx950
 * kernels (tests/, __graft_entry__.smoke()) and the CPU-baseline leg of
 * bench.py. Nothing in the product calls it.
 *
 * Every function computes in double over double arrays (inputs are the
 * exact FP32/FP16 values widened). Each follows the reference Triton kernel
 * named beside it (python/cutriton/triton_kernels/...):
 *   ct_oracle_conv2d          resnet.py:88-114   (zero padding, dilation)
 *   ct_oracle_batch_norm      resnet.py:117-130  ((x-mean)/sqrt(var+eps)*scale+bias)
 *   ct_oracle_max_pool        resnet.py:159-182  (-inf outside the image; NaN never
 *                             selected; +0 above -0)
 *   ct_oracle_global_avg_pool resnet.py:185-198  (sum / (H*W))
 *   ct_oracle_gemm            resnet.py:201-213, transformer.py:17-60 (+ bias[n])
 *   ct_oracle_gelu            transformer.py:110-116 (0.5 x (1 + erf(x/sqrt 2)))
 *   ct_oracle_layer_norm      transformer.py:128-177 (optional residual;
 *                             two-pass mean / centred variance; eps inside sqrt)
 *   ct_oracle_softmax         transformer.py:180-190 (last axis; subtract the
 *                             row max, exp, divide by the sum)
 *   ct_oracle_attention       no reference kernel: the ONNX Attention
 *                             operator's definition (softmax(scale Q K^T) V,
 *                             upper-left causal mask), built from the
 *                             softmax above
 * Parity pins (closed forms, invariants, brute force, torch float64) are in
 * tests/test_oracle.py.
 */
#include <math.h>
#include <stddef.h>
#include <stdlib.h>
#include <stdint.h>
#include <string.h>

void ct_oracle_conv2d(const double* x, int n, int c, int h, int w, const double* weight, int k, int r, int s,
                      int stride_h, int stride_w, int pad_h, int pad_w, int dil_h, int dil_w, int out_h,
                      int out_w, double* out) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int img = 0; img < n; ++img) {
    for (int oc = 0; oc < k; ++oc) {
      double* plane = out + ((size_t)img * k + oc) * out_h * out_w;
      memset(plane, 0, sizeof(double) * (size_t)out_h * out_w);
      for (int ic = 0; ic < c; ++ic) {
        const double* src = x + ((size_t)img * c + ic) * h * w;
        for (int kh = 0; kh < r; ++kh) {
          for (int kw = 0; kw < s; ++kw) {
            const double wv = weight[(((size_t)oc * c + ic) * r + kh) * s + kw];
            if (wv == 0.0) continue;
            for (int oh = 0; oh < out_h; ++oh) {
              const int ih = oh * stride_h - pad_h + kh * dil_h;
              if (ih < 0 || ih >= h) continue;
              const double* line = src + (size_t)ih * w;
              double* dst = plane + (size_t)oh * out_w;
              for (int ow = 0; ow < out_w; ++ow) {
                const int iw = ow * stride_w - pad_w + kw * dil_w;
                if (iw >= 0 && iw < w) dst[ow] += wv * line[iw];
              }
            }
          }
        }
      }
    }
  }
}

void ct_oracle_batch_norm(const double* x, int n, int c, long spatial, const double* scale, const double* bias,
                          const double* mean, const double* var, double eps, double* out) {
  for (long img = 0; img < n; ++img) {
    for (int ch = 0; ch < c; ++ch) {
      const double inv = 1.0 / sqrt(var[ch] + eps);
      const size_t base = ((size_t)img * c + ch) * spatial;
      for (long i = 0; i < spatial; ++i) out[base + i] = (x[base + i] - mean[ch]) * inv * scale[ch] + bias[ch];
    }
  }
}

void ct_oracle_max_pool(const double* x, int n, int c, int h, int w, int kernel_h, int kernel_w, int stride_h,
                        int stride_w, int pad_h, int pad_w, int dil_h, int dil_w, int out_h, int out_w,
                        double* out) {
  for (long plane = 0; plane < (long)n * c; ++plane) {
    const double* src = x + (size_t)plane * h * w;
    for (int oh = 0; oh < out_h; ++oh) {
      for (int ow = 0; ow < out_w; ++ow) {
        double best = -INFINITY;
        for (int kh = 0; kh < kernel_h; ++kh) {
          const int ih = oh * stride_h - pad_h + kh * dil_h;
          if (ih < 0 || ih >= h) continue;
          for (int kw = 0; kw < kernel_w; ++kw) {
            const int iw = ow * stride_w - pad_w + kw * dil_w;
            if (iw < 0 || iw >= w) continue;
            const double v = src[(size_t)ih * w + iw];
            /* tl.maximum(accumulator, v) of resnet.py:178-180 (maxNum: a NaN
             * never wins, so an all-NaN window keeps the -inf start); a tie of
             * zeros takes +0 (IEEE 754-2019 maximumNumber; maxNum leaves it
             * unspecified). */
            if (v > best || (v == 0.0 && best == 0.0 && signbit(best) && !signbit(v))) best = v;
          }
        }
        out[((size_t)plane * out_h + oh) * out_w + ow] = best;
      }
    }
  }
}

void ct_oracle_global_avg_pool(const double* x, long planes, long spatial, double* out) {
  for (long p = 0; p < planes; ++p) {
    double sum = 0.0;
    for (long i = 0; i < spatial; ++i) sum += x[(size_t)p * spatial + i];
    out[p] = sum / (double)spatial;
  }
}

/* out[m][n] = sum_k a[m][k] * b[k][n] (+ bias[n] when bias is non-null). */
void ct_oracle_gemm(const double* a, const double* b, const double* bias, int m, int n, int k, double* out) {
#pragma omp parallel for schedule(static)
  for (int i = 0; i < m; ++i) {
    double* row = out + (size_t)i * n;
    for (int j = 0; j < n; ++j) row[j] = bias ? bias[j] : 0.0;
    for (int t = 0; t < k; ++t) {
      const double av = a[(size_t)i * k + t];
      const double* brow = b + (size_t)t * n;
      for (int j = 0; j < n; ++j) row[j] += av * brow[j];
    }
  }
}

void ct_oracle_gelu(const double* x, long count, double* out) {
  for (long i = 0; i < count; ++i) out[i] = 0.5 * x[i] * (1.0 + erf(x[i] / sqrt(2.0)));
}

void ct_oracle_layer_norm(const double* x, const double* residual, long rows, long cols, const double* gamma,
                          const double* beta, double eps, double* out) {
  for (long r = 0; r < rows; ++r) {
    const double* xr = x + (size_t)r * cols;
    const double* rr = residual ? residual + (size_t)r * cols : NULL;
    double* yr = out + (size_t)r * cols;
    double mean = 0.0;
    for (long j = 0; j < cols; ++j) mean += xr[j] + (rr ? rr[j] : 0.0);
    mean /= (double)cols;
    double var = 0.0;
    for (long j = 0; j < cols; ++j) {
      const double d = xr[j] + (rr ? rr[j] : 0.0) - mean;
      var += d * d;
    }
    var /= (double)cols;
    const double inv = 1.0 / sqrt(var + eps);
    for (long j = 0; j < cols; ++j) yr[j] = (xr[j] + (rr ? rr[j] : 0.0) - mean) * inv * gamma[j] + beta[j];
  }
}

/* Row softmax over the last axis: e_j = exp(x_j - max_i x_i), y_j = e_j / sum e.
 * A row of -inf entries gives NaN (-inf - -inf), as the reference does. */
void ct_oracle_softmax(const double* x, long rows, long cols, double* out) {
  for (long r = 0; r < rows; ++r) {
    const double* xr = x + (size_t)r * cols;
    double* yr = out + (size_t)r * cols;
    double max = -INFINITY;
    for (long j = 0; j < cols; ++j) max = xr[j] > max ? xr[j] : max;
    double sum = 0.0;
    for (long j = 0; j < cols; ++j) {
      yr[j] = exp(xr[j] - max);
      sum += yr[j];
    }
    for (long j = 0; j < cols; ++j) yr[j] /= sum;
  }
}

/* Attention over `heads` independent [s_q, d] x [s_k, d] problems:
 * out[i] = sum_j softmax_j(scale * q[i] . k[j]) v[j], with `causal` keeping
 * only keys j <= i (upper-left alignment, as the ONNX Attention operator
 * and torch's scaled_dot_product_attention define is_causal). */
void ct_oracle_attention(const double* q, const double* k, const double* v, long heads, long s_q, long s_k, long d,
                         double scale, int causal, double* out) {
  double* logits = (double*)malloc((size_t)(s_k > 0 ? s_k : 1) * sizeof(double));
  double* weights = (double*)malloc((size_t)(s_k > 0 ? s_k : 1) * sizeof(double));
  for (long h = 0; h < heads; ++h) {
    const double* qh = q + (size_t)h * s_q * d;
    const double* kh = k + (size_t)h * s_k * d;
    const double* vh = v + (size_t)h * s_k * d;
    double* oh = out + (size_t)h * s_q * d;
    for (long i = 0; i < s_q; ++i) {
      for (long j = 0; j < s_k; ++j) {
        double dot = 0.0;
        for (long e = 0; e < d; ++e) dot += qh[(size_t)i * d + e] * kh[(size_t)j * d + e];
        logits[j] = (causal && j > i) ? -INFINITY : scale * dot;
      }
      ct_oracle_softmax(logits, 1, s_k, weights);
      for (long e = 0; e < d; ++e) {
        double acc = 0.0;
        for (long j = 0; j < s_k; ++j) acc += weights[j] * vh[(size_t)j * d + e];
        oh[(size_t)i * d + e] = acc;
      }
    }
  }
  free(logits);
  free(weights);
}

