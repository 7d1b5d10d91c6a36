/*
 * zn_hip.h -- C ABI of the MI355X (gfx950) fp32 GEMM backend for ZigNeuron.
 *
 * This is the drop-in boundary a Zig `HipBackend` binds with `extern fn`
 * declarations (zig/hip.zig holds them).  It replaces the
 * reference's CUDA stack for the GEMM path: the driver binding
 * (src/cuda_driver.zig:632-931), NVRTC (src/cuda_nvrtc.zig), the device
 * context (src/cuda_context.zig:382-1820) and the CudaBackend GEMM wrappers
 * (src/cuda.zig:521-797, 1008-1071, 2255-2338).  All citations are to the
 * reference tree.
 *
 * Conventions
 *  - Every function returns an int status: ZN_OK (0) or a negative ZN_ERR_*.
 *    Nothing aborts or throws across the boundary.
 *  - Matrices are row-major fp32.  The host-slice entry points take the
 *    reference's implicit leading dimensions (glossary of src/backend.zig:
 *    NN lda=K ldb=N; TN A stored [K x M]; NT B stored [N x K]; ldc=N); the
 *    device entry points take explicit leading dimensions and batch strides.
 *  - One context serves one host thread (the reference's Backend is not
 *    thread-safe, src/backend.zig:25).  Work is ordered on the context's one
 *    HIP stream.  Device-pointer entry points are asynchronous; host-slice
 *    entry points return only after the result is in host memory, like
 *    CudaBackend.matMul's final download (src/cuda.zig:617).
 *  - GEMM kernels are loaded from offline-built gfx950 code objects
 *    (zn_gemm_gfx950.hsaco); there is no runtime compilation and no CPU
 *    fallback: a missing device or code object is an error.
 */
#ifndef ZN_HIP_H
#define ZN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZN_HIP_ABI_VERSION 1

/* Status codes; zn_hip_status_string() names them.  Mapped to a Zig error set
 * the way checkCuda maps CUresult (src/cuda_driver.zig:1119-1160). */
#define ZN_OK 0
#define ZN_ERR_NO_DEVICE (-1)   /* no HIP device / not a gfx950 device */
#define ZN_ERR_CODE_OBJECT (-2) /* code object missing, unreadable or not loadable */
#define ZN_ERR_SYMBOL (-3)      /* a kernel symbol is missing from the code object */
#define ZN_ERR_INVALID_ARG (-4) /* null pointer, bad enum, short slice, bad leading dim */
#define ZN_ERR_OOM (-5)         /* device allocation failed */
#define ZN_ERR_LAUNCH (-6)      /* kernel launch failed */
#define ZN_ERR_HIP (-7)         /* other HIP runtime error; see zn_hip_last_hip_error */
#define ZN_ERR_OVERFLOW (-8)    /* a size product overflows, or exceeds the 32-bit index range */

/* Operand layouts (row-major storage). */
typedef enum zn_layout {
    ZN_LAYOUT_NN = 0, /* C[MxN] = A[MxK] . B[KxN]           (Backend.matMul)          */
    ZN_LAYOUT_NT = 1, /* C[MxN] = A[MxK] . B^T, B is [NxK]  (Backend.matMulTransposeB) */
    ZN_LAYOUT_TN = 2  /* C[MxN] = A^T . B[KxN], A is [KxM]  (Backend.matMulTransposeA) */
} zn_layout;

/* Epilogue activations, applied after the full K sum and the bias
 * (src/backend.zig:200-295; src/activation.zig:97-120). */
typedef enum zn_act {
    ZN_ACT_LINEAR = 0,  /* identity                                   */
    ZN_ACT_RELU = 1,    /* v > 0 ? v : 0                              */
    ZN_ACT_SIGMOID = 2, /* 1/(1+exp(-v)) fused; branch-stable elementwise */
    ZN_ACT_TANH = 3     /* tanh(v)                                    */
} zn_act;

typedef struct zn_ctx zn_ctx;
typedef struct zn_event zn_event;
typedef struct zn_graph zn_graph;

typedef struct zn_device_info {
    char name[64];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int32_t compute_units;  /* multiProcessorCount */
    int32_t clock_khz;      /* max engine clock */
    int64_t total_mem;      /* bytes of HBM */
} zn_device_info;

/* ---------------------------------------------------------------- context */

/* ABI version of the loaded library (ZN_HIP_ABI_VERSION). */
int zn_hip_abi_version(void);

/* 1 when at least one HIP device is visible, else 0.  Replaces
 * CudaBackend.isAvailable (src/cuda.zig:317-328) for Backend.detect
 * (src/backend.zig:84-94). */
int zn_hip_available(void);

/* Create a context on `device`: select the device, create one stream, load
 * the gfx950 code object from `code_object_dir` (NULL: $ZN_HIP_CODE_OBJECT_DIR,
 * else the directory holding this library) and resolve every kernel symbol.
 * Replaces CudaBackend.init -> CudaContext.init -> loadBuiltinKernels
 * (src/cuda.zig:163-300, src/cuda_context.zig:382-497, 1325-1414). */
int zn_hip_create(int device, const char *code_object_dir, zn_ctx **out);

/* Synchronize, release cached device memory, unload the module, destroy the
 * stream and free the context (CudaBackend.deinit).  NULL is a no-op. */
int zn_hip_destroy(zn_ctx *ctx);

/* Static string naming a status code. */
const char *zn_hip_status_string(int status);

/* The hipError_t behind the last ZN_ERR_HIP / ZN_ERR_OOM / ZN_ERR_LAUNCH on ctx. */
int zn_hip_last_hip_error(const zn_ctx *ctx);

/* Device properties (CudaContext.queryDeviceProperties, src/cuda_context.zig:713). */
int zn_hip_device_info(const zn_ctx *ctx, zn_device_info *out);

/* The context's hipStream_t, for callers that order their own work with it. */
void *zn_hip_stream(const zn_ctx *ctx);

/* ----------------------------------------------------------------- memory */

/* Caller-owned device buffers (256-byte aligned).  Replace
 * CudaContext.getBuffer / returnBuffer for device-resident callers
 * (src/cuda_context.zig:773-852). */
int zn_hip_alloc(zn_ctx *ctx, size_t bytes, void **out);
int zn_hip_free(zn_ctx *ctx, void *ptr);
/* Blocking copies (CudaContext.upload / download, src/cuda_context.zig:882-920). */
int zn_hip_h2d(zn_ctx *ctx, void *dst, const void *src, size_t bytes);
int zn_hip_d2h(zn_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Stream-ordered copies; host memory must stay valid until zn_hip_sync. */
int zn_hip_h2d_async(zn_ctx *ctx, void *dst, const void *src, size_t bytes);
int zn_hip_d2h_async(zn_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Fill `count` floats with `value` using a kernel (safe under graph capture). */
int zn_hip_fill_f32(zn_ctx *ctx, float *dst, float value, int64_t count);
/* Device-to-device copy of `count` floats with a plain streaming kernel. */
int zn_hip_copy_f32(zn_ctx *ctx, float *dst, const float *src, int64_t count);
/* Keep the context's stream busy for `microseconds` (at most 100000) with a
 * one-wave kernel that sleeps on the device clock.  No counterpart in the
 * reference: a measurement aid for timing small kernels, so that launches
 * queued behind it run back to back from the device queue, whatever the
 * host's submission rate. */
int zn_hip_hold_stream(zn_ctx *ctx, float microseconds);
/* Wait for all work on the context's stream. */
int zn_hip_sync(zn_ctx *ctx);

/* ----------------------------------------------------------------- graphs */

/* Capture the device-pointer calls that follow on the context's stream into a
 * HIP graph (stream capture, relaxed mode) instead of running them; replay it
 * with one launch.  No counterpart in the reference: it serves callers whose
 * steps are bound by launch cost, such as a small-batch MLP training step.
 *  - Calls that wait for the device (zn_hip_sync, zn_hip_free, blocking
 *    copies, the *_host drop-ins) return ZN_ERR_INVALID_ARG while capturing.
 *  - Run the sequence once before capturing it: a GEMM that would have to
 *    grow the split-K workspace during capture runs unsplit instead.
 *  - Buffers the runtime leases during capture belong to the graph until
 *    zn_hip_graph_destroy; graphs still alive are destroyed by zn_hip_destroy.
 *  - Nothing in a graph clears memory with a memset node (fills are kernels). */
int zn_hip_graph_begin(zn_ctx *ctx);
int zn_hip_graph_end(zn_ctx *ctx, zn_graph **out);
int zn_hip_graph_launch(zn_ctx *ctx, zn_graph *graph);
/* Waits for the context's stream, then releases the graph and its buffers. */
int zn_hip_graph_destroy(zn_graph *graph);

/* ----------------------------------------------------------------- events */

/* HIP events on the context's stream, for kernel timing (the role of the
 * cuEvent timing in CudaContext.launchKernel, src/cuda_context.zig:1711-1772). */
int zn_hip_event_create(zn_ctx *ctx, zn_event **out);
int zn_hip_event_record(zn_ctx *ctx, zn_event *ev);
/* Milliseconds between two recorded events; waits for `end`. */
int zn_hip_event_elapsed_ms(zn_event *start, zn_event *end, float *ms);
int zn_hip_event_destroy(zn_event *ev);

/* ------------------------------------------------ GEMM on device pointers */

/* Macro-tile override for the GEMM launch policy: ZN_TILE_AUTO (the default)
 * picks by problem size; the others force one tile for every following GEMM
 * on this context.  No counterpart in the reference: it exists for tuning and
 * for tests that must reach every kernel variant. */
#define ZN_TILE_AUTO (-1)
#define ZN_TILE_256x128 0
#define ZN_TILE_128x128 1
#define ZN_TILE_128x64 2
#define ZN_TILE_64x64 3
#define ZN_TILE_32x32 4
#define ZN_TILE_128x128_K32 5 /* 128x128, BK 32, one workgroup per CU; not for convolutions */
#define ZN_TILE_64x64_K16 6   /* 64x64, BK 16, six workgroups per CU; not for convolutions */
#define ZN_TILE_256x256 7     /* 256x256, BK 16, one workgroup per CU; 16-byte rows only (otherwise 256x128); not for
                                 convolutions */
int zn_hip_set_gemm_tile(zn_ctx *ctx, int tile);
/* Split-K override: 0 (the default) lets the policy choose, 1..256 asks for
 * that many K slices (at most ceil(K / BK)) for every following GEMM on this
 * context; K is cut into equal slices of whole BK multiples, which can give
 * fewer.  Like the tile override, a tuning and test hook with no reference
 * counterpart. */
int zn_hip_set_gemm_splits(zn_ctx *ctx, int splits);
/* Persistent-kernel override: -1 (the default) lets the policy choose, 0
 * never uses the persistent GEMM kernels, 1 uses them for every eligible
 * GEMM (unsplit, 16-byte staging, K > 0, a tile other than 32x32) without
 * deferred stores, 2 the same with deferred stores wherever those apply
 * (plain GEMMs on 128x128 tiles that all lie inside C, K > 48; the policy
 * uses them too).  Results are bit-identical in every mode.  A tuning and
 * test hook with no reference counterpart. */
int zn_hip_set_gemm_persistent(zn_ctx *ctx, int mode);
/* Intra-workgroup split-K override: -1 (the default) lets the policy choose
 * (problems of at most one 32x32 tile per CU, 64 <= K <= 4096), 0 never
 * uses it, 4 or 8 runs every GEMM with K > 0 (other than the convolutions')
 * on 32x32 tiles whose 4 or 8 waves split K and sum their partial tiles in
 * wave order, 16 on 16x16 tiles whose 4 waves do the same.  A tuning and
 * test hook with no reference counterpart. */
int zn_hip_set_gemm_wave_split(zn_ctx *ctx, int waves);

/* C = act((accumulate ? C : 0) + op(A).op(B) + bias) for one problem.
 * `bias` (length N) may be NULL.  Leading dimensions are in elements and must
 * be >= the stored row length.  m, n >= 0; k >= 0 (k == 0 gives the epilogue
 * of a zero sum).  Asynchronous on the context stream.
 * Generalises CudaBackend.matMul(a,b,c,m,n,k,transpose_a,transpose_b,accumulate)
 * (src/cuda.zig:540-618) and matMulBiasActivation (src/cuda.zig:1008-1071). */
int zn_hip_sgemm(zn_ctx *ctx, int layout, int64_t m, int64_t n, int64_t k, const float *a, int64_t lda,
                 const float *b, int64_t ldb, float *c, int64_t ldc, int accumulate, const float *bias, int act);

/* zn_hip_sgemm without any allocation: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * results as zn_hip_sgemm, except:
 *  - split-K partial sums go to a fixed 64 MiB per-device scratch array in
 *    the library (held until the process ends) instead of the context's
 *    growable workspace.  When the launch policy's split would need more,
 *    the GEMM runs unsplit; a split forced with zn_hip_set_gemm_splits that
 *    needs more is refused with ZN_ERR_INVALID_ARG;
 *  - operands are never copied into padded rows: rows that are not whole
 *    16-byte float4s are staged with 4-byte loads (the same result).
 * Results equal zn_hip_sgemm's bit for bit whenever both split K alike.
 * Nothing in the scratch needs clearing between calls (each slice writes all
 * of its partial sums).  All contexts on one device share its scratch: a
 * call made by another context than the device's previous one first makes
 * its stream wait (on the device, hipStreamWaitEvent) for that call's
 * kernels, so calls from different contexts and threads run one after the
 * other; the host does not block.  Calls made under stream capture are not
 * ordered so: replays of a graph that holds one must not overlap other
 * no-allocation calls on the device.  Returns ZN_ERR_OOM or ZN_ERR_HIP if
 * the scratch could not be set up when the context was created (the next
 * context created on the device tries again). */
int zn_hip_sgemm_noalloc(zn_ctx *ctx, int layout, int64_t m, int64_t n, int64_t k, const float *a, int64_t lda,
                         const float *b, int64_t ldb, float *c, int64_t ldc, int accumulate, const float *bias,
                         int act);

/* `batch` independent problems; operand p of problem i starts at
 * p + i*stride_p (elements).  stride_a or stride_b may be 0 (a shared
 * operand, as in CudaBackend.matMulBatch's shared B, src/cuda.zig:729-797).
 * Attention QK^T / PV and im2col convolution GEMMs use this entry
 * (src/cuda.zig:2255-2281, 3026-3100). */
int zn_hip_sgemm_strided_batched(zn_ctx *ctx, int layout, int64_t m, int64_t n, int64_t k, const float *a,
                                 int64_t lda, int64_t stride_a, const float *b, int64_t ldb, int64_t stride_b,
                                 float *c, int64_t ldc, int64_t stride_c, int64_t batch, int accumulate,
                                 const float *bias, int act);

/* ------------------------------------ Dense helpers on device pointers */

/* out[r*n + i] += bias[i]  (Backend.addBias, src/backend.zig:658-671). */
int zn_hip_add_bias(zn_ctx *ctx, float *out, const float *bias, int64_t rows, int64_t n);
/* Activation.forward per element (Backend.activationForward, src/backend.zig:367-386). */
int zn_hip_activation_forward(zn_ctx *ctx, int act, const float *in, float *out, int64_t len);
/* grad_in = grad_out * act'(y) from the activated output y
 * (Backend.activationBackward, src/backend.zig:390-399, src/optimization.zig:229-303). */
int zn_hip_activation_backward(zn_ctx *ctx, int act, const float *y, const float *grad_out, float *grad_in,
                               int64_t len);
/* grad_bias[i] += sum over rows r (ascending) of gaa[r*n + i]
 * (Backend.accumulateBias, src/backend.zig:649-655, 706-713). */
int zn_hip_accumulate_bias(zn_ctx *ctx, float *grad_bias, const float *gaa, int64_t rows, int64_t n);

/* Dense.backward (src/layer.zig:411-475) on device pointers, row-major
 * input [batch x in], weights [in x out], activated_output / grad_output /
 * grad_after_act [batch x out]:
 *   grad_after_act = activationBackward(act, activated_output, grad_output)
 *   grad_bias     += column sums of grad_after_act          (accumulateBias)
 *   grad_input     = grad_after_act . weights^T             (matMulTransposeB)
 *   grad_weights   = input^T . grad_after_act  (overwritten) (matMulTransposeA)
 * The first two run as one pass; the bias sums are taken over row splits and
 * added in split order (deterministic, within the GEMM tolerance rather than
 * bit-identical to the row-by-row sum of zn_hip_accumulate_bias).
 * grad_input may be null to skip it. */
int zn_hip_dense_backward(zn_ctx *ctx, int act, const float *input, const float *weights,
                          const float *activated_output, const float *grad_output, float *grad_after_act,
                          float *grad_input, float *grad_weights, float *grad_bias, int64_t batch, int64_t in_size,
                          int64_t out_size);
/* zn_hip_dense_backward for a stack of Dense layers walked top-down, with
 * fewer launches.  No counterpart in the reference, whose backward loop
 * (src/network.zig:455-477) calls Dense.backward layer by layer; this gives
 * the same bits as zn_hip_dense_backward called that way.
 *   gaa_ready = 1: grad_after_act already holds this layer's derivative
 *     (written by the layer above's call); activated_output and grad_output
 *     are not read and may be null.
 *   prev_grad_after_act != null: also writes the layer below's
 *     prev_grad_after_act = activationBackward(prev_act,
 *     prev_activated_output, grad_input) (grad_input must be non-null), so
 *     that layer's call can pass gaa_ready = 1.
 * Results are bit-identical to zn_hip_dense_backward on the same layers. */
int zn_hip_dense_backward_chain(zn_ctx *ctx, int act, const float *input, const float *weights,
                                const float *activated_output, const float *grad_output, float *grad_after_act,
                                float *grad_input, float *grad_weights, float *grad_bias, int64_t batch,
                                int64_t in_size, int64_t out_size, int gaa_ready, int prev_act,
                                const float *prev_activated_output, float *prev_grad_after_act);

/* Two stacked Dense layers, the lower one [in -> hidden] (x, W1 [in x hidden],
 * b1, act1) and the top one [hidden -> out] (W2 [hidden x out], b2, act2),
 * with a launch that spans both layers when the top layer has at most 16
 * outputs (a classifier head).  The reference runs the same work layer by
 * layer: Network.forward calls Dense.forward per layer
 * (src/network.zig:309-360, src/layer.zig:380-409), and its backward loop
 * calls Dense.backward per layer, top first (src/network.zig:455-477,
 * src/layer.zig:411-475).  Sizes as Dense.init requires: in, hidden and out
 * of at least 1 (ZN_ERR_INVALID_ARG otherwise, src/layer.zig:304-305).
 *
 * Forward: h = act1(x . W1 + b1) [batch x hidden], y = act2(h . W2 + b2)
 * [batch x out], as Backend.matMulBias* computes each (src/backend.zig:
 * 200-295), within the GEMM tolerance.  b1 and b2 may be null (no bias). */
int zn_hip_dense_pair_forward(zn_ctx *ctx, int act1, const float *x, const float *w1, const float *b1, float *h,
                              int act2, const float *w2, const float *b2, float *y, int64_t batch, int64_t in_size,
                              int64_t hidden, int64_t out_size);
/* Backward of the pair, from grad_y [batch x out]:
 *   gaa2 = activationBackward(act2, y, grad_y), grad_h = gaa2 . W2^T,
 *   grad_w2 = h^T . gaa2 (overwritten), grad_b2 += column sums of gaa2;
 *   gaa1 = activationBackward(act1, h, grad_h), grad_x = gaa1 . W1^T
 *   (skipped when grad_x is null), grad_w1 = x^T . gaa1 (overwritten),
 *   grad_b1 += column sums of gaa1.
 * y is read only for a non-linear act2.  gaa2 and gaa1 are
 * activationBackward's bits on y and on the grad_h written; the GEMMs are
 * within the GEMM tolerance, and the bias sums are deterministic, within it. */
int zn_hip_dense_pair_backward(zn_ctx *ctx, int act1, const float *x, const float *w1, const float *h, float *gaa1,
                               float *grad_x, float *grad_w1, float *grad_b1, int act2, const float *w2,
                               const float *y, const float *grad_y, float *gaa2, float *grad_h, float *grad_w2,
                               float *grad_b2, int64_t batch, int64_t in_size, int64_t hidden, int64_t out_size);

/* ------------------------------------- conv and attention (device pointers) */

/* Backend.im2col (src/backend.zig:3775-3827) on device: NCHW `input` ->
 * col[(b*OH*OW + oh*OW + ow)][(kh*kW + kw)*C + ic], zero in the padding. */
int zn_hip_im2col(zn_ctx *ctx, const float *input, float *col, int64_t batch, int64_t channels, int64_t in_h,
                  int64_t in_w, int64_t k_h, int64_t k_w, int64_t out_h, int64_t out_w, int64_t stride_h,
                  int64_t stride_w, int64_t pad_h, int64_t pad_w);
/* cpuConv2dForwardIm2col (src/backend.zig:3881-3950) on device, as an
 * implicit GEMM: per image out[OC][OH*OW] = W . im2col(input)^T + bias[oc]
 * (NCHW output), the im2col operand gathered on the fly (no col buffer).
 * Like the reference, W is read as [OC][(kh*kW + kw)*C + ic], the K order of
 * the im2col columns. */
int zn_hip_conv2d_forward_im2col(zn_ctx *ctx, const float *input, const float *weights, const float *bias,
                                 float *output, int64_t batch, int64_t in_channels, int64_t out_channels, int64_t k_h,
                                 int64_t k_w, int64_t in_h, int64_t in_w, int64_t out_h, int64_t out_w,
                                 int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w);
/* The same implicit GEMM with W read as [OC][C][kH][kW]: the convolution of
 * the direct branch of cpuConv2dForward (src/backend.zig:3019-3041). */
int zn_hip_conv2d_forward_direct(zn_ctx *ctx, const float *input, const float *weights, const float *bias,
                                 float *output, int64_t batch, int64_t in_channels, int64_t out_channels, int64_t k_h,
                                 int64_t k_w, int64_t in_h, int64_t in_w, int64_t out_h, int64_t out_w,
                                 int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w);
/* Backend.col2im (src/backend.zig:3833-3877) on device: NCHW output = the sum
 * of the col entries [(b*OH*OW + oh*OW + ow)][(kh*kW + kw)*C + ic] landing on
 * each pixel, added in the reference's order (bit-identical); output is
 * overwritten. */
int zn_hip_col2im(zn_ctx *ctx, const float *col, float *output, int64_t batch, int64_t channels, int64_t in_h,
                  int64_t in_w, int64_t k_h, int64_t k_w, int64_t out_h, int64_t out_w, int64_t stride_h,
                  int64_t stride_w, int64_t pad_h, int64_t pad_w);
/* cpuConv2dBackwardIm2col (src/backend.zig:3954-4065) on device.  Like the
 * reference, grad_output is read as [batch*OH*OW][OC] by the weight and input
 * gradients (grad_weights = go^T . im2col(input), grad_input =
 * col2im(go . W), W and grad_weights in the col K order) and as NCHW by
 * grad_bias (the per-channel sum).  All three outputs are overwritten. */
int zn_hip_conv2d_backward_im2col(zn_ctx *ctx, const float *input, const float *weights, const float *grad_output,
                                  float *grad_input, float *grad_weights, float *grad_bias, int64_t batch,
                                  int64_t in_channels, int64_t out_channels, int64_t k_h, int64_t k_w, int64_t in_h,
                                  int64_t in_w, int64_t out_h, int64_t out_w, int64_t stride_h, int64_t stride_w,
                                  int64_t pad_h, int64_t pad_w);
/* The direct branch of cpuConv2dBackward (src/backend.zig:3064-3094) on
 * device: NCHW grad_output, weights and grad_weights as [OC][C][kH][kW]
 * (the gradients of zn_hip_conv2d_forward_direct).  Outputs overwritten. */
int zn_hip_conv2d_backward_direct(zn_ctx *ctx, const float *input, const float *weights, const float *grad_output,
                                  float *grad_input, float *grad_weights, float *grad_bias, int64_t batch,
                                  int64_t in_channels, int64_t out_channels, int64_t k_h, int64_t k_w, int64_t in_h,
                                  int64_t in_w, int64_t out_h, int64_t out_w, int64_t stride_h, int64_t stride_w,
                                  int64_t pad_h, int64_t pad_w);
/* Row softmax of scaled scores (out may equal in): out[r,:] = exp(s - max) /
 * sum(exp(s - max)), s = in[r,:] * scale, the softmax of cpuAttentionForward
 * (src/backend.zig:3201-3214). */
int zn_hip_softmax_rows(zn_ctx *ctx, const float *in, float *out, int64_t rows, int64_t n, float scale);
/* cpuAttentionForward (src/backend.zig:3197-3222) for `batch` independent
 * single-head problems [seq_len x d_k] laid out back to back (e.g. B*H heads
 * of a [B,H,S,D] tensor): out = softmax(scale * Q.K^T) . V.  For d_k <= 128
 * one fused kernel streams K and V past each block of queries (online
 * softmax) and never writes the scores; larger d_k run QK^T (NT GEMM), the
 * row softmax and P.V (NN GEMM) with batch*seq_len^2 scores taken from the
 * context's buffer cache. */
int zn_hip_attention_forward(zn_ctx *ctx, const float *q, const float *k, const float *v, float *out, int64_t batch,
                             int64_t seq_len, int64_t d_k, float scale);

/* ------------------------------- Backend drop-ins on host slices (sync) */
/* Each takes the reference method's slices as (pointer, length) pairs and its
 * scalar arguments unchanged, stages through the context's cached device
 * buffers, and returns when `c` holds the result.  A slice shorter than the
 * shape requires is ZN_ERR_INVALID_ARG. */

/* Backend.matMul (src/backend.zig:169-182): C[m x n] (+)= A[m x k] . B[k x n]. */
int zn_hip_mat_mul(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len, float *c,
                   size_t c_len, size_t m, size_t n, size_t k, int accumulate);
/* Backend.matMulBatch (src/backend.zig:186-195): rows of A against a shared B. */
int zn_hip_mat_mul_batch(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len, float *c,
                         size_t c_len, size_t batch_size, size_t n, size_t k, int accumulate);
/* Backend.matMulTransposeA (src/backend.zig:298-307): C = A^T . B, A is [k x m]. */
int zn_hip_mat_mul_transpose_a(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len, float *c,
                               size_t c_len, size_t m, size_t n, size_t k, int accumulate);
/* Backend.matMulTransposeB (src/backend.zig:310-325): C = A . B^T, B is [n x k]. */
int zn_hip_mat_mul_transpose_b(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len, float *c,
                               size_t c_len, size_t m, size_t n, size_t k, int accumulate);
/* Backend.matMulBias (src/backend.zig:200-222). */
int zn_hip_mat_mul_bias(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len, const float *bias,
                        size_t bias_len, float *c, size_t c_len, size_t batch_size, size_t n, size_t k);
/* Backend.matMulBiasRelu (src/backend.zig:225-247). */
int zn_hip_mat_mul_bias_relu(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len,
                             const float *bias, size_t bias_len, float *c, size_t c_len, size_t batch_size, size_t n,
                             size_t k);
/* Backend.matMulBiasSigmoid (src/backend.zig:250-272). */
int zn_hip_mat_mul_bias_sigmoid(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len,
                                const float *bias, size_t bias_len, float *c, size_t c_len, size_t batch_size,
                                size_t n, size_t k);
/* Backend.matMulBiasTanh (src/backend.zig:275-295). */
int zn_hip_mat_mul_bias_tanh(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len,
                             const float *bias, size_t bias_len, float *c, size_t c_len, size_t batch_size, size_t n,
                             size_t k);
/* Backend.addBias (src/backend.zig:658-671): rows = out_len / bias_len. */
int zn_hip_add_bias_host(zn_ctx *ctx, float *out, size_t out_len, const float *bias, size_t bias_len);
/* Backend.activationForward (src/backend.zig:367-386) for linear/relu/sigmoid/tanh. */
int zn_hip_activation_forward_host(zn_ctx *ctx, int act, const float *in, size_t in_len, float *out,
                                   size_t out_len);
/* Backend.activationBackward (src/backend.zig:390-399) for linear/relu/sigmoid/tanh. */
int zn_hip_activation_backward_host(zn_ctx *ctx, int act, const float *y, size_t y_len, const float *grad_out,
                                    size_t grad_out_len, float *grad_in, size_t grad_in_len);
/* Backend.accumulateBias (src/backend.zig:649-655): rows = gaa_len / grad_bias_len. */
int zn_hip_accumulate_bias_host(zn_ctx *ctx, float *grad_bias, size_t grad_bias_len, const float *gaa,
                                size_t gaa_len);

/* Backend.conv2dForward (src/backend.zig:507-518 -> cpuConv2dForward :3004):
 * batch = input_len / (C*H*W).  Keeps the reference's switch: when
 * batch*OC*OH*OW >= 1024 and kH*kW >= 9 the weights are read in the im2col
 * K order (cpuConv2dForwardIm2col), otherwise as [OC][C][kH][kW] (the direct
 * branch); both run as the implicit GEMM on the device. */
int zn_hip_conv2d_forward_host(zn_ctx *ctx, const float *input, size_t input_len, const float *weights,
                               size_t weights_len, const float *bias, size_t bias_len, float *output,
                               size_t output_len, size_t in_channels, size_t out_channels, size_t k_h, size_t k_w,
                               size_t in_h, size_t in_w, size_t out_h, size_t out_w, size_t stride_h, size_t stride_w,
                               size_t pad_h, size_t pad_w);
/* Backend.conv2dBackward (src/backend.zig:520, CPU arm :3049-3095): batch =
 * input_len / (C*H*W); the im2col branch (zn_hip_conv2d_backward_im2col) when
 * batch*OC*OH*OW >= 1024 and kH*kW >= 9, the direct branch otherwise. */
int zn_hip_conv2d_backward_host(zn_ctx *ctx, const float *input, size_t input_len, const float *weights,
                                size_t weights_len, const float *grad_output, size_t grad_output_len,
                                float *grad_input, size_t grad_input_len, float *grad_weights, size_t grad_weights_len,
                                float *grad_bias, size_t grad_bias_len, size_t in_channels, size_t out_channels,
                                size_t k_h, size_t k_w, size_t in_h, size_t in_w, size_t out_h, size_t out_w,
                                size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w);
/* Backend.attentionForward (src/backend.zig:631-638): one head [seq_len x
 * d_k]; `scores` (length >= seq_len, as the reference requires) is not
 * written: the device keeps its scores in HBM. */
int zn_hip_attention_forward_host(zn_ctx *ctx, const float *q, size_t q_len, const float *k, size_t k_len,
                                  const float *v, size_t v_len, float *output, size_t output_len, float *scores,
                                  size_t scores_len, size_t seq_len, size_t d_k, float scale);

#ifdef __cplusplus
}
#endif
#endif /* ZN_HIP_H */
