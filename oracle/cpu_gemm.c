/*
 * oracle/cpu_gemm.c -- TEST INFRASTRUCTURE ONLY (the parity checker and the
 * timed CPU baseline).  Never linked into, loaded by or called from the
 * product library; the product path fails loudly when its HIP code objects
 * are missing instead of falling back here.
 *
 * A plain-C restatement of ZigNeuron's CPU GEMM family.  The reference is
 * Zig, which cannot be compiled in this image (no zig toolchain), so this
 * restatement *is* the oracle.  Bit-exactness argument: in every reference
 * loop the value of C[i,j] is built by p = 0..K-1 ascending steps of
 * fl(fl(c) + fl(a*b)) (Zig's default float mode never contracts to FMA), and
 * IEEE round-to-nearest-even fp32 SSE arithmetic with -ffp-contract=off does
 * exactly the same.  Loop blocking only changes *when* each step happens,
 * never the per-element order, so all branches agree bit-for-bit.
 *
 * Pins (tests/test_oracle.py): the reference's known-answer tests
 * (tests/golden/reference_kats.json), exact integer matmuls against numpy's
 * int64 matmul, the NN/TN/NT transpose identities (bit-exact), a vectorised
 * float32 sequential-order restatement (bit-exact), fp64 error bounds, and
 * closed forms for the epilogues, im2col and attention.  Zig's own f32
 * exp/tanh rounding (std.math.exp / std.math.tanh, ported musl code) is not
 * reproduced bit-for-bit: libm expf/tanhf are used and the epilogue tests
 * bound them against fp64 to a few ulp ("parity unpinned" at ulp level only).
 */
#include "cpu_gemm.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ZNO_BLOCK 32 /* block_size in src/backend.zig:2522 */

static size_t zno_min(size_t x, size_t y) { return x < y ? x : y; }

/* One 32-row block band [i0, i1) of the blocked branch: kk outer, jj inner,
 * then rows, then p, then the contiguous j run (src/backend.zig:2525-2569).
 * The reference's Vec8 fast path (aligned rows) computes c + a*b lane-wise,
 * identical to the scalar statement below. */
static void zno_blocked_band(const float *a, const float *b, float *c, size_t i0, size_t i1, size_t n,
                             size_t k) {
    for (size_t kk = 0; kk < k; kk += ZNO_BLOCK) {
        const size_t k_end = zno_min(kk + ZNO_BLOCK, k);
        for (size_t jj = 0; jj < n; jj += ZNO_BLOCK) {
            const size_t j_end = zno_min(jj + ZNO_BLOCK, n);
            for (size_t i = i0; i < i1; ++i) {
                float *crow = c + i * n;
                for (size_t p = kk; p < k_end; ++p) {
                    const float av = a[i * k + p];
                    const float *brow = b + p * n;
                    for (size_t j = jj; j < j_end; ++j) {
                        const float prod = av * brow[j];
                        crow[j] = crow[j] + prod;
                    }
                }
            }
        }
    }
}

void zno_matmul_blocked(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate) {
    if (!accumulate) memset(c, 0, m * n * sizeof(float));
    for (size_t ii = 0; ii < m; ii += ZNO_BLOCK) zno_blocked_band(a, b, c, ii, zno_min(ii + ZNO_BLOCK, m), n, k);
}

void zno_matmul_blocked_omp(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate,
                            int threads) {
    if (!accumulate) memset(c, 0, m * n * sizeof(float));
    const long nblk = (long)((m + ZNO_BLOCK - 1) / ZNO_BLOCK);
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (long blk = 0; blk < nblk; ++blk) {
        const size_t ii = (size_t)blk * ZNO_BLOCK;
        zno_blocked_band(a, b, c, ii, zno_min(ii + ZNO_BLOCK, m), n, k);
    }
}

/* i-p-j saxpy order (src/backend.zig:2571-2606). */
void zno_matmul_unblocked(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate) {
    if (!accumulate) memset(c, 0, m * n * sizeof(float));
    for (size_t i = 0; i < m; ++i) {
        float *crow = c + i * n;
        for (size_t p = 0; p < k; ++p) {
            const float av = a[i * k + p];
            const float *brow = b + p * n;
            for (size_t j = 0; j < n; ++j) {
                const float prod = av * brow[j];
                crow[j] = crow[j] + prod;
            }
        }
    }
}

/* cpuMatMul: the blocked branch only when every dimension reaches the block
 * size (src/backend.zig:2523). */
void zno_matmul(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate) {
    if (m >= ZNO_BLOCK && n >= ZNO_BLOCK && k >= ZNO_BLOCK)
        zno_matmul_blocked(a, b, c, m, n, k, accumulate);
    else
        zno_matmul_unblocked(a, b, c, m, n, k, accumulate);
}

/* cpuMatMulBatch: row i runs cpuMatMul(a + i*k, b, c + i*n, 1, n, k), whose
 * non-accumulating memset clears the whole remaining slice c[i*n ..]
 * (src/backend.zig:2609-2613 with :2521). */
void zno_matmul_batch(const float *a, const float *b, float *c, size_t batch, size_t n, size_t k, int accumulate) {
    for (size_t i = 0; i < batch; ++i) {
        float *crow = c + i * n;
        if (!accumulate) memset(crow, 0, (batch - i) * n * sizeof(float));
        /* m = 1 < 32, so cpuMatMul takes the unblocked branch; the memset
         * has just been done above for the full tail. */
        for (size_t p = 0; p < k; ++p) {
            const float av = a[i * k + p];
            const float *brow = b + p * n;
            for (size_t j = 0; j < n; ++j) {
                const float prod = av * brow[j];
                crow[j] = crow[j] + prod;
            }
        }
    }
}

/* Dot-product loops shared by TN and NT: sum starts at 0, runs p ascending,
 * then C = sum or C += sum (src/backend.zig:2615-2647). */
static void zno_tn_rows(const float *a, const float *b, float *c, size_t i0, size_t i1, size_t m, size_t n,
                        size_t k, int accumulate) {
    for (size_t i = i0; i < i1; ++i)
        for (size_t j = 0; j < n; ++j) {
            float sum = 0.0f;
            for (size_t p = 0; p < k; ++p) {
                const float prod = a[p * m + i] * b[p * n + j];
                sum = sum + prod;
            }
            c[i * n + j] = accumulate ? c[i * n + j] + sum : sum;
        }
}

static void zno_nt_rows(const float *a, const float *b, float *c, size_t i0, size_t i1, size_t n, size_t k,
                        int accumulate) {
    for (size_t i = i0; i < i1; ++i)
        for (size_t j = 0; j < n; ++j) {
            float sum = 0.0f;
            for (size_t p = 0; p < k; ++p) {
                const float prod = a[i * k + p] * b[j * k + p];
                sum = sum + prod;
            }
            c[i * n + j] = accumulate ? c[i * n + j] + sum : sum;
        }
}

void zno_matmul_tn(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate) {
    zno_tn_rows(a, b, c, 0, m, m, n, k, accumulate);
}

void zno_matmul_nt(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate) {
    zno_nt_rows(a, b, c, 0, m, n, k, accumulate);
}

void zno_matmul_tn_omp(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate,
                       int threads) {
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (long i = 0; i < (long)m; ++i) zno_tn_rows(a, b, c, (size_t)i, (size_t)i + 1, m, n, k, accumulate);
}

void zno_matmul_nt_omp(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate,
                       int threads) {
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (long i = 0; i < (long)m; ++i) zno_nt_rows(a, b, c, (size_t)i, (size_t)i + 1, n, k, accumulate);
}

/* src/activation.zig:97-99 */
static float zno_relu(float x) { return x > 0.0f ? x : 0.0f; }
/* Branch-stable sigmoid of Activation.forward (src/activation.zig:105-112). */
static float zno_sigmoid_stable(float x) {
    if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
    const float e = expf(x);
    return e / (1.0f + e);
}

void zno_matmul_bias_act(const float *a, const float *b, const float *bias, float *c, size_t batch, size_t n,
                         size_t k, int act) {
    zno_matmul_batch(a, b, c, batch, n, k, 0);
    for (size_t r = 0; r < batch; ++r)
        for (size_t j = 0; j < n; ++j) {
            const float v = c[r * n + j] + bias[j];
            float out = v;
            switch (act) {
            case ZNO_ACT_RELU: out = v > 0.0f ? v : 0.0f; break;                /* :239-240 */
            case ZNO_ACT_SIGMOID: out = 1.0f / (1.0f + expf(-v)); break;        /* :264-265 */
            case ZNO_ACT_TANH: out = tanhf(v); break;                           /* :289-290 */
            default: break;                                                     /* :215 */
            }
            c[r * n + j] = out;
        }
}

void zno_add_bias(float *out, size_t out_len, const float *bias, size_t bias_len) {
    const size_t rows = out_len / bias_len; /* batch_size = output.len / bias.len */
    for (size_t r = 0; r < rows; ++r)
        for (size_t i = 0; i < bias_len; ++i) out[r * bias_len + i] = out[r * bias_len + i] + bias[i];
}

void zno_activation_forward(int act, const float *in, float *out, size_t len) {
    for (size_t i = 0; i < len; ++i) {
        const float x = in[i];
        switch (act) {
        case ZNO_ACT_RELU: out[i] = zno_relu(x); break;
        case ZNO_ACT_SIGMOID: out[i] = zno_sigmoid_stable(x); break;
        case ZNO_ACT_TANH: out[i] = tanhf(x); break; /* src/activation.zig:118-120 */
        default: out[i] = x; break;                  /* .linear, :29 */
        }
    }
}

/* src/optimization.zig:229-303: relu passes grad where y > 0; sigmoid
 * go*y*(1-y) evaluated left to right; tanh go*(1-y*y); linear copies. */
void zno_activation_backward(int act, const float *y, const float *grad_out, float *grad_in, size_t len) {
    for (size_t i = 0; i < len; ++i) {
        const float yi = y[i], go = grad_out[i];
        switch (act) {
        case ZNO_ACT_RELU: grad_in[i] = yi > 0.0f ? go : 0.0f; break;
        case ZNO_ACT_SIGMOID: {
            const float t = go * yi;
            grad_in[i] = t * (1.0f - yi);
            break;
        }
        case ZNO_ACT_TANH: {
            const float yy = yi * yi;
            grad_in[i] = go * (1.0f - yy);
            break;
        }
        default: grad_in[i] = go; break;
        }
    }
}

void zno_accumulate_bias(float *grad_bias, size_t n, const float *gaa, size_t gaa_len) {
    const size_t rows = gaa_len / n;
    for (size_t r = 0; r < rows; ++r)
        for (size_t i = 0; i < n; ++i) grad_bias[i] = grad_bias[i] + gaa[r * n + i];
}

void zno_im2col(const float *input, float *col, size_t batch, size_t channels, size_t in_h, size_t in_w,
                size_t k_h, size_t k_w, size_t out_h, size_t out_w, size_t stride_h, size_t stride_w,
                size_t pad_h, size_t pad_w) {
    const size_t col_h = out_h * out_w, col_w = k_h * k_w * channels;
    memset(col, 0, batch * col_h * col_w * sizeof(float));
    for (size_t bi = 0; bi < batch; ++bi)
        for (size_t oh = 0; oh < out_h; ++oh)
            for (size_t ow = 0; ow < out_w; ++ow) {
                float *dst = col + (bi * col_h + oh * out_w + ow) * col_w;
                const long h0 = (long)(oh * stride_h) - (long)pad_h;
                const long w0 = (long)(ow * stride_w) - (long)pad_w;
                for (size_t ic = 0; ic < channels; ++ic)
                    for (size_t kh = 0; kh < k_h; ++kh)
                        for (size_t kw = 0; kw < k_w; ++kw) {
                            const long ih = h0 + (long)kh, iw = w0 + (long)kw;
                            if (ih < 0 || iw < 0 || ih >= (long)in_h || iw >= (long)in_w) continue;
                            dst[(kh * k_w + kw) * channels + ic] =
                                input[((bi * channels + ic) * in_h + (size_t)ih) * in_w + (size_t)iw];
                        }
            }
}

void zno_conv2d_im2col_gemm(const float *col, const float *weights, const float *bias, float *out, size_t batch,
                            size_t out_channels, size_t col_height, size_t col_width) {
    const size_t vec_end = (col_width / 4) * 4;
    for (size_t bi = 0; bi < batch; ++bi)
        for (size_t hw = 0; hw < col_height; ++hw) {
            const float *row = col + (bi * col_height + hw) * col_width;
            for (size_t oc = 0; oc < out_channels; ++oc) {
                const float *w = weights + oc * col_width;
                float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                size_t i = 0;
                for (; i < vec_end; i += 4)
                    for (int l = 0; l < 4; ++l) {
                        const float prod = row[i + (size_t)l] * w[i + (size_t)l];
                        lane[l] = lane[l] + prod;
                    }
                float sum = 0.0f;
                float red = lane[0] + lane[1];
                red = red + lane[2];
                red = red + lane[3];
                sum = sum + red;
                for (; i < col_width; ++i) {
                    const float prod = row[i] * w[i];
                    sum = sum + prod;
                }
                out[(bi * out_channels + oc) * col_height + hw] = sum + bias[oc];
            }
        }
}

void zno_conv2d_forward(const float *input, size_t input_len, const float *weights, const float *bias, float *out,
                        size_t channels, size_t out_channels, size_t k_h, size_t k_w, size_t in_h, size_t in_w,
                        size_t out_h, size_t out_w, size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w) {
    const size_t batch = input_len / (channels * in_h * in_w);
    const size_t total_out = batch * out_channels * out_h * out_w;
    if (total_out >= 1024 && k_h * k_w >= 9) {
        const size_t col_h = out_h * out_w, col_w = k_h * k_w * channels;
        float *col = (float *)malloc(batch * col_h * col_w * sizeof(float));
        if (!col) return;
        zno_im2col(input, col, batch, channels, in_h, in_w, k_h, k_w, out_h, out_w, stride_h, stride_w, pad_h,
                   pad_w);
        zno_conv2d_im2col_gemm(col, weights, bias, out, batch, out_channels, col_h, col_w);
        free(col);
        return;
    }
    for (size_t bi = 0; bi < batch; ++bi)
        for (size_t oc = 0; oc < out_channels; ++oc)
            for (size_t oh = 0; oh < out_h; ++oh)
                for (size_t ow = 0; ow < out_w; ++ow) {
                    float sum = 0.0f;
                    const long h0 = (long)(oh * stride_h) - (long)pad_h;
                    const long w0 = (long)(ow * stride_w) - (long)pad_w;
                    for (size_t ic = 0; ic < channels; ++ic)
                        for (size_t kh = 0; kh < k_h; ++kh)
                            for (size_t kw = 0; kw < k_w; ++kw) {
                                const long ih = h0 + (long)kh, iw = w0 + (long)kw;
                                if (ih < 0 || iw < 0 || ih >= (long)in_h || iw >= (long)in_w) continue;
                                const float prod =
                                    input[((bi * channels + ic) * in_h + (size_t)ih) * in_w + (size_t)iw] *
                                    weights[((oc * channels + ic) * k_h + kh) * k_w + kw];
                                sum = sum + prod;
                            }
                    out[((bi * out_channels + oc) * out_h + oh) * out_w + ow] = sum + bias[oc];
                }
}

void zno_col2im(const float *col, float *output, size_t batch, size_t channels, size_t in_h, size_t in_w,
                size_t k_h, size_t k_w, size_t out_h, size_t out_w, size_t stride_h, size_t stride_w,
                size_t pad_h, size_t pad_w) {
    const size_t col_h = out_h * out_w, col_w = k_h * k_w * channels;
    memset(output, 0, batch * channels * in_h * in_w * sizeof(float));
    for (size_t bi = 0; bi < batch; ++bi)
        for (size_t oh = 0; oh < out_h; ++oh)
            for (size_t ow = 0; ow < out_w; ++ow) {
                const float *src = col + (bi * col_h + oh * out_w + ow) * col_w;
                const long h0 = (long)(oh * stride_h) - (long)pad_h;
                const long w0 = (long)(ow * stride_w) - (long)pad_w;
                for (size_t ic = 0; ic < channels; ++ic)
                    for (size_t kh = 0; kh < k_h; ++kh)
                        for (size_t kw = 0; kw < k_w; ++kw) {
                            const long ih = h0 + (long)kh, iw = w0 + (long)kw;
                            if (ih < 0 || iw < 0 || ih >= (long)in_h || iw >= (long)in_w) continue;
                            float *dst = output + ((bi * channels + ic) * in_h + (size_t)ih) * in_w + (size_t)iw;
                            *dst = *dst + src[(kh * k_w + kw) * channels + ic];
                        }
            }
}

void zno_conv2d_backward_direct(const float *input, const float *weights, const float *grad_output, float *grad_input,
                                float *grad_weights, float *grad_bias, size_t batch, size_t channels,
                                size_t out_channels, size_t k_h, size_t k_w, size_t in_h, size_t in_w, size_t out_h,
                                size_t out_w, size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w) {
    memset(grad_input, 0, batch * channels * in_h * in_w * sizeof(float));
    memset(grad_weights, 0, out_channels * channels * k_h * k_w * sizeof(float));
    memset(grad_bias, 0, out_channels * sizeof(float));
    for (size_t bi = 0; bi < batch; ++bi)
        for (size_t oc = 0; oc < out_channels; ++oc)
            for (size_t oh = 0; oh < out_h; ++oh)
                for (size_t ow = 0; ow < out_w; ++ow) {
                    const float go = grad_output[((bi * out_channels + oc) * out_h + oh) * out_w + ow];
                    grad_bias[oc] = grad_bias[oc] + go;
                    const long h0 = (long)(oh * stride_h) - (long)pad_h;
                    const long w0 = (long)(ow * stride_w) - (long)pad_w;
                    for (size_t ic = 0; ic < channels; ++ic)
                        for (size_t kh = 0; kh < k_h; ++kh)
                            for (size_t kw = 0; kw < k_w; ++kw) {
                                const long ih = h0 + (long)kh, iw = w0 + (long)kw;
                                if (ih < 0 || iw < 0 || ih >= (long)in_h || iw >= (long)in_w) continue;
                                const size_t in_idx = ((bi * channels + ic) * in_h + (size_t)ih) * in_w + (size_t)iw;
                                const size_t w_idx = ((oc * channels + ic) * k_h + kh) * k_w + kw;
                                const float pw = input[in_idx] * go;
                                grad_weights[w_idx] = grad_weights[w_idx] + pw;
                                const float pi = weights[w_idx] * go;
                                grad_input[in_idx] = grad_input[in_idx] + pi;
                            }
                }
}

void zno_conv2d_backward_im2col(const float *input, const float *weights, const float *grad_output, float *grad_input,
                                float *grad_weights, float *grad_bias, size_t batch, size_t channels,
                                size_t out_channels, size_t k_h, size_t k_w, size_t in_h, size_t in_w, size_t out_h,
                                size_t out_w, size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w) {
    const size_t col_h = out_h * out_w, col_w = k_h * k_w * channels, rows = batch * col_h;
    float *col = (float *)malloc(rows * col_w * sizeof(float));
    float *grad_col = (float *)malloc(rows * col_w * sizeof(float));
    if (!col || !grad_col) {
        free(col);
        free(grad_col);
        return;
    }
    memset(grad_weights, 0, out_channels * col_w * sizeof(float));
    memset(grad_bias, 0, out_channels * sizeof(float));
    zno_im2col(input, col, batch, channels, in_h, in_w, k_h, k_w, out_h, out_w, stride_h, stride_w, pad_h, pad_w);
    for (size_t bi = 0; bi < batch; ++bi)
        for (size_t oc = 0; oc < out_channels; ++oc)
            for (size_t hw = 0; hw < col_h; ++hw)
                grad_bias[oc] = grad_bias[oc] + grad_output[(bi * out_channels + oc) * col_h + hw];
    for (size_t r = 0; r < rows; ++r)
        for (size_t oc = 0; oc < out_channels; ++oc) {
            const float go = grad_output[r * out_channels + oc];
            float *gw = grad_weights + oc * col_w;
            const float *cr = col + r * col_w;
            for (size_t i = 0; i < col_w; ++i) {
                const float prod = cr[i] * go;
                gw[i] = gw[i] + prod;
            }
        }
    memset(grad_col, 0, rows * col_w * sizeof(float));
    for (size_t r = 0; r < rows; ++r)
        for (size_t oc = 0; oc < out_channels; ++oc) {
            const float go = grad_output[r * out_channels + oc];
            const float *w = weights + oc * col_w;
            float *gc = grad_col + r * col_w;
            for (size_t i = 0; i < col_w; ++i) {
                const float prod = w[i] * go;
                gc[i] = gc[i] + prod;
            }
        }
    zno_col2im(grad_col, grad_input, batch, channels, in_h, in_w, k_h, k_w, out_h, out_w, stride_h, stride_w, pad_h,
               pad_w);
    free(col);
    free(grad_col);
}

void zno_conv2d_backward(const float *input, size_t input_len, const float *weights, const float *grad_output,
                         float *grad_input, float *grad_weights, float *grad_bias, size_t channels,
                         size_t out_channels, size_t k_h, size_t k_w, size_t in_h, size_t in_w, size_t out_h,
                         size_t out_w, size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w) {
    const size_t batch = input_len / (channels * in_h * in_w);
    const size_t total_out = batch * out_channels * out_h * out_w;
    if (total_out >= 1024 && k_h * k_w >= 9)
        zno_conv2d_backward_im2col(input, weights, grad_output, grad_input, grad_weights, grad_bias, batch, channels,
                                   out_channels, k_h, k_w, in_h, in_w, out_h, out_w, stride_h, stride_w, pad_h, pad_w);
    else
        zno_conv2d_backward_direct(input, weights, grad_output, grad_input, grad_weights, grad_bias, batch, channels,
                                   out_channels, k_h, k_w, in_h, in_w, out_h, out_w, stride_h, stride_w, pad_h, pad_w);
}

void zno_attention(const float *q, const float *k, const float *v, float *out, float *scores, size_t seq_len,
                   size_t d_k, float scale) {
    for (size_t i = 0; i < seq_len; ++i) {
        float mx = -INFINITY;
        for (size_t m = 0; m < seq_len; ++m) {
            float s = 0.0f;
            for (size_t f = 0; f < d_k; ++f) {
                const float prod = q[i * d_k + f] * k[m * d_k + f];
                s = s + prod;
            }
            s = s * scale;
            scores[m] = s;
            if (s > mx) mx = s;
        }
        float total = 0.0f;
        for (size_t m = 0; m < seq_len; ++m) {
            scores[m] = expf(scores[m] - mx);
            total = total + scores[m];
        }
        for (size_t f = 0; f < d_k; ++f) {
            float r = 0.0f;
            for (size_t m = 0; m < seq_len; ++m) {
                const float prod = (scores[m] / total) * v[m * d_k + f];
                r = r + prod;
            }
            out[i * d_k + f] = r;
        }
    }
}
