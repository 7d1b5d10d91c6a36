// Kernel argument blocks shared by the host runtime (zn_hip.cpp) and the
// gfx950 code objects (kernels/*.hip).  Each kernel takes one of these structs
// by value, so the host passes a single kernel parameter whose layout is fixed
// here.  Plain C layout; no HIP types.
#ifndef ZN_KERNEL_ARGS_H
#define ZN_KERNEL_ARGS_H

#include <stdint.h>

// Geometry of an implicit-GEMM convolution operand: B[k][n] is the im2col
// element of output pixel n = oh*out_w + ow and filter tap k, gathered from
// the NCHW input of one image (blockIdx.y).
struct ZnConvGeom {
    int32_t channels, in_h, in_w, k_h, k_w, out_w;
    int32_t stride_h, stride_w, pad_h, pad_w;
    int32_t k_order;  // 0: k = (kh*k_w + kw)*channels + ic (im2col order); 1: k = (ic*k_h + kh)*k_w + kw (OIHW)
    // Unsigned division by a constant for 0 <= x < 2^31: x / d ==
    // (x * mul) >> (31 + shift) with shift = ceil(log2 d), mul = ceil(2^(31 + shift) / d).
    // div1 splits k into its outer and inner index (channels for k_order 0,
    // k_h*k_w for 1); the other divisors are k_w and out_w.
    int32_t div1;
    uint32_t div1_mul, div1_shift, kw_mul, kw_shift, ow_mul, ow_shift;
    // Weight gradient only (K runs over the pixels of `images` images):
    // out_h and its divisor.
    int32_t out_h, images;
    uint32_t oh_mul, oh_shift;
    // NHWC forward only: 1 when every K slice lies in one filter tap
    // (channels a multiple of the tile's BK).
    int32_t tap_uniform;
};

// One (possibly batched) fp32 GEMM: C = act((acc ? C : 0) + op(A) op(B) + bias).
struct ZnGemmArgs {
    const float *a;
    const float *b;
    float *c;
    const float *bias;   // length n, or null
    int64_t lda, ldb, ldc;
    int64_t stride_a, stride_b, stride_c;  // batch strides (elements); batch = blockIdx.y
    int32_t m, n, k;
    int32_t tiles_m, tiles_n;  // macro-tile grid of one problem; gridDim.x == tiles_m * tiles_n
    int32_t accumulate;        // 1: add the existing C
    int32_t act;               // zn_act
    int32_t vec_c;             // 1: ldc and C allow vector stores
    int32_t group_m;           // tile rows per raster group
    int32_t xcd_remap;         // 1: gridDim.x % 8 == 0, give each XCD a contiguous tile range;
                               // 2: split-K with gridDim.y == 1, each XCD a contiguous (slice, tile) range;
                               // 3: deferred-store persistent kernels, each XCD a contiguous run of work items
    // split-K: blockIdx.z = slice of K; splits > 1 writes raw partial sums to
    // ws[(problem * splits + slice)][m][n] and a reduce kernel finishes C.
    int32_t splits;
    int32_t k_chunk;           // K per slice, a multiple of the tile's BK
    float *ws;
    int32_t bias_rows;         // 1: bias is indexed by row (length m), else by column (length n)
    int32_t batch;             // problems; the persistent kernels walk batch * tiles_m * tiles_n work items
    ZnConvGeom conv;           // the zn_conv_* kernels only
    // Chained activation derivative (intra-workgroup split-K tiles only):
    // when chain_gaa is set, each finished element v of C also gives
    // chain_gaa[i] = act'(chain_y[i]) * v (act = chain_act), both laid out like C.
    const float *chain_y;
    float *chain_gaa;
    int32_t chain_act;
    // Intra-workgroup split-K kernels with splits > 1: one counter per
    // (problem, tile), kCounterStride ints apart, zero between launches (the
    // last workgroup of a tile resets it).
    int32_t *counters;
    // Row tail folded into the launch (the unaligned 128x128 kernels,
    // batch 1): tail_rows more rows of C after row m, A's rows (TN: columns)
    // from tail_a, C's from tail_c (row stride ldc); each element is one
    // K-long dot product, and workgroup w (over blockIdx.x and .z) computes
    // elements [w * tail_per_wg, (w + 1) * tail_per_wg) in row-major order.
    // The bias (by row: entries m ..) and the epilogue are those of the main
    // rows.  tail_per_wg <= 4, K <= 1024.
    const float *tail_a;
    float *tail_c;
    int32_t tail_rows, tail_per_wg;
};

// Cross-workgroup arrival counters (the context's counter array): counter i
// sits at index i * kCounterStride, one 128-byte line each, so that arrivals
// at different counters do not contend for one line (the atomics of one line
// are serialised where they execute).
constexpr int kCounterStride = 32;

// Split-K reduction: C = act((accumulate ? C : 0) + sum_s ws[s] + bias), the
// slices summed in ascending order.
struct ZnReduceArgs {
    const float *ws;
    float *c;
    const float *bias;
    int64_t ldc, stride_c;
    int32_t m, n, batch, splits;
    int32_t accumulate, act, vec;
    int32_t bias_rows;
};

// Bias gradient as column sums in one launch: dst[c] += sum over row splits
// s (ascending) of (sum over the split's rows r, ascending, of src[r*n + c]),
// splits of `per` rows; the same sums as zn_dense_grad_prologue's partials
// added by the split-K reduce.  copy (optional) receives src.
constexpr int kMaxColSumSplits = 256;  // row splits the grouped launches' column sums take

struct ZnColSumArgs {
    const float *src;
    float *dst;
    float *copy;
    int32_t rows, n, per, splits;
};

// The GEMMs of one Dense backward in one launch: workgroups [0, wg_nt)
// compute grad_input (NT), the next wg_tn grad_weights (TN), and the last
// ones the bias gradient: wg_bias reduce the partial sums a prologue wrote
// (the prologue also wrote grad_after_act), or, without a prologue,
// wg_colsum sum the columns of grad_after_act themselves.
struct ZnDenseBwdArgs {
    ZnGemmArgs nt;
    ZnGemmArgs tn;
    ZnReduceArgs bias;     // reduce of the prologue's partial sums (wg_bias workgroups), or
    ZnColSumArgs colsum;   // the column sums themselves (wg_colsum workgroups)
    int32_t wg_nt, wg_tn, wg_bias, wg_colsum;
};

// Two stacked Dense layers whose top layer is narrow (out <= 16), forward
// in one launch: h = act1(x . W1 + b1) on the 16x16 wave-split tiles (l1,
// activation in l1.act); each tile's block of h times W2's matching rows is
// its partial sum of the strip's y, and the last tile to finish each 16-row
// strip adds the strip's partials into y = act2(h . W2 + b2).
struct ZnPairFwdArgs {
    ZnGemmArgs l1;
    const float *w2;      // [hidden x out]
    const float *b2;      // [out], or null
    float *y;             // [batch x out]
    float *part;          // 256 floats per tile: its 16 x 16 partial sum of y
    int32_t *counters;    // one per 16-row strip of h, kCounterStride ints apart, zero between launches
    int32_t out, act2;
};

// One GEMM of the pair backward on 32x32 tiles: C [m x n] (row stride ldc)
// over K = k, with one operand staged from `src` (row stride ld) and the
// other generated in registers.
struct ZnPairGemm {
    const float *src;
    float *c;
    int32_t ld, ldc, m, n, k, tiles_n;
};

// The backward of the same pair in one launch.  gaa2 = act2'(y, grad_y),
// grad_h = gaa2 . W2^T and gaa1 = act1'(h, grad_h) are generated where they
// are needed (no workgroup waits for another):
//   [0, wg_nt)    grad_x  = gaa1 . W1^T on 32x64 tiles (nt: W1 staged; none when grad_x is null)
//   next wg_tn1   grad_w1 = x^T . gaa1 on 32x32 tiles (tn1: x staged); the tiles of a column
//                 share the writes of its grad_h and gaa1, and the first row of tiles adds
//                 gaa1's column sums into grad_b1
//   next wg_tn2   grad_w2 = h^T . gaa2 (tn2: h staged); the first tile also writes gaa2 and
//                 adds its column sums into grad_b2
struct ZnPairBwdArgs {
    ZnPairGemm nt, tn1, tn2;
    const float *h;       // [batch x hidden], the lower layer's activated output
    const float *w2;      // [hidden x out]
    const float *y;       // [batch x out], the top layer's activated output (read unless act2 is linear)
    const float *grad_y;  // [batch x out]
    float *gaa1, *grad_h, *gaa2, *grad_b1, *grad_b2;
    int32_t batch, hidden, out, act1, act2;
    int32_t wg_nt, wg_tn1, wg_tn2;
};

// Elementwise helpers (fill, copy, bias, activations, bias gradient, row
// softmax).
struct ZnEltArgs {
    float *out;
    const float *in0;
    const float *in1;
    int64_t rows, n;   // n = row length; for flat ops rows*n = element count
    float value;       // fill value; softmax score scale
    int32_t act;
};

// Fused attention: per problem blockIdx.y, out = softmax(scale * q k^T) v
// over [seq_len x d_k] row-major heads `stride` floats apart.
struct ZnAttnArgs {
    const float *q;
    const float *k;
    const float *v;
    float *out;
    int64_t stride;
    int32_t seq_len, d_k;
    float scale_log2;  // scale * log2(e): scores are exponentiated base 2
};

// Dense backward prologue: gaa = act'(y) * grad_out elementwise and, per
// split of `rows_per_split` rows (blockIdx.y), the column sums of gaa.
struct ZnDenseGradArgs {
    const float *y;        // activated output [rows x n]
    const float *go;       // grad_output [rows x n]
    float *gaa;            // grad after activation [rows x n]; null: only the sums
    float *partial;        // [splits x n] column sums
    int64_t rows, n;
    int32_t act;
    int32_t rows_per_split;
};

// im2col / col2im: col[(b*OH*OW + oh*OW + ow)][tap], tap = (kh*KW + kw)*C + ic
// (k_order 0, the Backend.im2col layout) or (ic*KH + kh)*KW + kw (k_order 1,
// the OIHW weight order).
struct ZnIm2colArgs {
    float *image;  // NCHW: read by im2col, written by col2im
    float *col;    // written by im2col, read by col2im
    int32_t batch, channels, in_h, in_w, k_h, k_w, out_h, out_w, stride_h, stride_w, pad_h, pad_w;
    int32_t k_order;
};

// Row packing: dst[r][c] = c < cols ? src[r * ld_src + c] : 0 for
// c < ld_dst (a multiple of 4, dst 16-byte aligned).
struct ZnPackArgs {
    const float *src;
    float *dst;
    int64_t rows, cols, ld_src, ld_dst;
};

// Up to two row packings in one launch: blockIdx.y selects op[blockIdx.y].
struct ZnPack2Args {
    ZnPackArgs op[2];
};

// Per image b < batch: dst_b[p][c] = src_b[c][p] for c < channels, p < pixels
// (NCHW -> NHWC).
struct ZnTransposeArgs {
    const float *src;
    float *dst;
    int64_t batch, channels, pixels;
};

// Weight regroup for the transposed-convolution input gradient:
// out[ic][t*OC + oc] = in[oc][t*C + ic] for t < taps_per_channel (kH*kW).
struct ZnRegroupArgs {
    const float *in;
    float *out;
    int32_t out_channels, channels, taps_per_channel;
};

#endif
