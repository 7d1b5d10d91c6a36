/*
 * oracle/cpu_gemm.h -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of ZigNeuron's CPU GEMM path (the reference's own `.cpu`
 * arms of `Backend.matMul*`).  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or as the timed CPU baseline -- never as the product path.
 *
 * All matrices are row-major fp32 with the reference's implicit leading
 * dimensions (lda = K or M, ldb = N or K, ldc = N).  Every function is built
 * with -ffp-contract=off and without -ffast-math so that each
 * c = c + a*b step rounds twice, exactly like Zig's strict float mode.
 */
#ifndef ZN_ORACLE_CPU_GEMM_H
#define ZN_ORACLE_CPU_GEMM_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Activation ids; same numbering as the product C-ABI (ZN_ACT_*). */
enum { ZNO_ACT_LINEAR = 0, ZNO_ACT_RELU = 1, ZNO_ACT_SIGMOID = 2, ZNO_ACT_TANH = 3 };

/* cpuMatMul, dispatching to the 32-blocked branch when m,n,k >= 32
 * (src/backend.zig:2520-2607). */
void zno_matmul(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate);
/* The unblocked i-p-j branch only (src/backend.zig:2571-2606). */
void zno_matmul_unblocked(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate);
/* The 32-blocked ii-kk-jj-i-p-j branch for any shape (src/backend.zig:2523-2570). */
void zno_matmul_blocked(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate);
/* Blocked branch with the ii row-block loop spread over `threads` OpenMP
 * threads; per-element K order is unchanged, so results are bit-identical. */
void zno_matmul_blocked_omp(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate, int threads);
/* cpuMatMulBatch: cpuMatMul(m=1) once per row, including the per-row memset
 * of the whole tail of C (src/backend.zig:2609-2613, 2521). */
void zno_matmul_batch(const float *a, const float *b, float *c, size_t batch, size_t n, size_t k, int accumulate);
/* cpuMatMulTransposeA: C = A^T B, A stored [K x M] (src/backend.zig:2615-2630). */
void zno_matmul_tn(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate);
/* cpuMatMulTransposeB: C = A B^T, B stored [N x K] (src/backend.zig:2632-2647). */
void zno_matmul_nt(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate);
/* OpenMP row-split twins of the TN / NT dot-product loops (bit-identical). */
void zno_matmul_tn_omp(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate, int threads);
void zno_matmul_nt_omp(const float *a, const float *b, float *c, size_t m, size_t n, size_t k, int accumulate, int threads);

/* matMulBias / matMulBiasRelu / matMulBiasSigmoid / matMulBiasTanh CPU
 * fallbacks (src/backend.zig:200-295): cpuMatMulBatch(acc=false), then per
 * element v = c + bias[col] and the activation (sigmoid as 1/(1+exp(-v)),
 * tanh as tanh(v)).  act = ZNO_ACT_LINEAR gives matMulBias. */
void zno_matmul_bias_act(const float *a, const float *b, const float *bias, float *c, size_t batch, size_t n, size_t k, int act);

/* Backend.addBias CPU arm: out[b*N+i] += bias[i] (src/backend.zig:658-671). */
void zno_add_bias(float *out, size_t out_len, const float *bias, size_t bias_len);
/* Activation.forward per element (src/activation.zig:24-35, 97-120). */
void zno_activation_forward(int act, const float *in, float *out, size_t len);
/* cpuActivationBackward for relu/sigmoid/tanh/linear
 * (src/backend.zig:2649-2662 -> src/optimization.zig:229-303). */
void zno_activation_backward(int act, const float *y, const float *grad_out, float *grad_in, size_t len);
/* cpuAccumulateBias: grad_bias[i] += sum_b gaa[b*N+i] (src/backend.zig:706-713). */
void zno_accumulate_bias(float *grad_bias, size_t n, const float *gaa, size_t gaa_len);

/* Backend.im2col (src/backend.zig:3775-3827): col[(b*OH*OW+oh*OW+ow) x (kh*kW+kw)*C+ic]. */
void zno_im2col(const float *input, float *col, size_t batch, size_t channels, size_t in_h, size_t in_w,
                size_t k_h, size_t k_w, size_t out_h, size_t out_w, size_t stride_h, size_t stride_w,
                size_t pad_h, size_t pad_w);
/* cpuConv2dForwardIm2col GEMM stage (src/backend.zig:3881-3950): per (b,hw,oc)
 * a 4-lane partial-sum dot of col row with W[oc,:], plus bias, NCHW output. */
void zno_conv2d_im2col_gemm(const float *col, const float *weights, const float *bias, float *out,
                            size_t batch, size_t out_channels, size_t col_height, size_t col_width);
/* cpuConv2dForward (src/backend.zig:3004-3045): batch = input_len / (C*H*W);
 * the im2col + GEMM stage when batch*OC*OH*OW >= 1024 and kH*kW >= 9 (weights
 * then read as [OC][(kh*kW+kw)*C+ic], like the reference), otherwise the
 * direct loop with weights [OC][C][kH][kW]. */
void zno_conv2d_forward(const float *input, size_t input_len, const float *weights, const float *bias, float *out,
                        size_t channels, size_t out_channels, size_t k_h, size_t k_w, size_t in_h, size_t in_w,
                        size_t out_h, size_t out_w, size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w);
/* Backend.col2im (src/backend.zig:3833-3877): output (NCHW) = 0, then every
 * in-image col element added at its input position, loops b, oh, ow, ic, kh, kw. */
void zno_col2im(const float *col, float *output, size_t batch, size_t channels, size_t in_h, size_t in_w,
                size_t k_h, size_t k_w, size_t out_h, size_t out_w, size_t stride_h, size_t stride_w,
                size_t pad_h, size_t pad_w);
/* The direct branch of cpuConv2dBackward (src/backend.zig:3064-3094): NCHW
 * grad_output, OIHW weights; grad_input, grad_weights, grad_bias overwritten. */
void zno_conv2d_backward_direct(const float *input, const float *weights, const float *grad_output, float *grad_input,
                                float *grad_weights, float *grad_bias, size_t batch, size_t channels,
                                size_t out_channels, size_t k_h, size_t k_w, size_t in_h, size_t in_w, size_t out_h,
                                size_t out_w, size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w);
/* cpuConv2dBackwardIm2col (src/backend.zig:3954-4065): grad_bias from the NCHW
 * grad_output; grad_weights[oc][c] = sum over rows r of col[r][c] *
 * grad_output[r*OC + oc] and grad_col[r][c] = sum over oc of W[oc][c] *
 * grad_output[r*OC + oc] (grad_output read as [batch*OH*OW][OC], weights in
 * the col K order); grad_input = col2im(grad_col). */
void zno_conv2d_backward_im2col(const float *input, const float *weights, const float *grad_output, float *grad_input,
                                float *grad_weights, float *grad_bias, size_t batch, size_t channels,
                                size_t out_channels, size_t k_h, size_t k_w, size_t in_h, size_t in_w, size_t out_h,
                                size_t out_w, size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w);
/* cpuConv2dBackward (src/backend.zig:3049-3095): batch = input_len / (C*H*W);
 * the im2col branch when batch*OC*OH*OW >= 1024 and kH*kW >= 9, else direct. */
void zno_conv2d_backward(const float *input, size_t input_len, const float *weights, const float *grad_output,
                         float *grad_input, float *grad_weights, float *grad_bias, size_t channels,
                         size_t out_channels, size_t k_h, size_t k_w, size_t in_h, size_t in_w, size_t out_h,
                         size_t out_w, size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w);
/* cpuAttentionForward (src/backend.zig:3197-3222), single head [S x D]. */
void zno_attention(const float *q, const float *k, const float *v, float *out, float *scores,
                   size_t seq_len, size_t d_k, float scale);

#ifdef __cplusplus
}
#endif
#endif
