// Elementwise and reduction helpers of the Dense path for gfx950:
// fill, copy (also the HBM reference kernel for counter calibration), bias
// add, activation forward/backward and the bias-gradient column sum.
// All are HBM-bound streaming kernels: coalesced, grid-stride, 16-byte
// accesses where alignment allows.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../zn_kernel_args.h"
#include "zn_activation.h"

typedef float zn_f32x4 __attribute__((ext_vector_type(4)));

namespace {

// Activation.forward (src/activation.zig:24-35, 97-120); sigmoid in the
// branch-stable form of src/activation.zig:105-112.
__device__ __forceinline__ float act_forward(float x, int act) {
    switch (act) {
    case 1: return x > 0.0f ? x : 0.0f;
    case 2:
        if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
        else {
            const float e = expf(x);
            return e / (1.0f + e);
        }
    case 3: return tanhf(x);
    default: return x;
    }
}


__device__ __forceinline__ int64_t gtid() { return (int64_t)blockIdx.x * blockDim.x + threadIdx.x; }
__device__ __forceinline__ int64_t gstride() { return (int64_t)gridDim.x * blockDim.x; }

}  // namespace

extern "C" __global__ __launch_bounds__(256) void zn_fill_f32(ZnEltArgs p) {
    const int64_t total = p.rows * p.n;
    for (int64_t i = gtid(); i < total; i += gstride()) p.out[i] = p.value;
}

// out[i] = in0[i]; dwordx4 body when both pointers are 16-byte aligned,
// four independent 16-byte loads in flight per thread before their stores.
extern "C" __global__ __launch_bounds__(256) void zn_copy_f32(ZnEltArgs p) {
    const int64_t total = p.rows * p.n;
    const bool aligned = ((reinterpret_cast<uintptr_t>(p.out) | reinterpret_cast<uintptr_t>(p.in0)) & 15) == 0;
    if (aligned) {
        const int64_t nv = total >> 2;
        const zn_f32x4 *src = reinterpret_cast<const zn_f32x4 *>(p.in0);
        zn_f32x4 *dst = reinterpret_cast<zn_f32x4 *>(p.out);
        const int64_t stride = gstride();
        int64_t i = gtid();
        for (; i + 3 * stride < nv; i += 4 * stride) {
            const zn_f32x4 v0 = __builtin_nontemporal_load(src + i);
            const zn_f32x4 v1 = __builtin_nontemporal_load(src + i + stride);
            const zn_f32x4 v2 = __builtin_nontemporal_load(src + i + 2 * stride);
            const zn_f32x4 v3 = __builtin_nontemporal_load(src + i + 3 * stride);
            __builtin_nontemporal_store(v0, dst + i);
            __builtin_nontemporal_store(v1, dst + i + stride);
            __builtin_nontemporal_store(v2, dst + i + 2 * stride);
            __builtin_nontemporal_store(v3, dst + i + 3 * stride);
        }
        for (; i < nv; i += stride) dst[i] = src[i];
        for (int64_t t = (nv << 2) + gtid(); t < total; t += stride) p.out[t] = p.in0[t];
    } else {
        for (int64_t i = gtid(); i < total; i += gstride()) p.out[i] = p.in0[i];
    }
}

// out[r*n + i] += bias[i]  (Backend.addBias, src/backend.zig:658-671).
extern "C" __global__ __launch_bounds__(256) void zn_add_bias(ZnEltArgs p) {
    const int64_t total = p.rows * p.n;
    for (int64_t i = gtid(); i < total; i += gstride()) p.out[i] = p.out[i] + p.in0[i % p.n];
}

extern "C" __global__ __launch_bounds__(256) void zn_activation_forward(ZnEltArgs p) {
    const int64_t total = p.rows * p.n;
    for (int64_t i = gtid(); i < total; i += gstride()) p.out[i] = act_forward(p.in0[i], p.act);
}

// in0 = activated output y, in1 = grad_out, out = grad_in.
extern "C" __global__ __launch_bounds__(256) void zn_activation_backward(ZnEltArgs p) {
    const int64_t total = p.rows * p.n;
    for (int64_t i = gtid(); i < total; i += gstride()) p.out[i] = zn_act_backward(p.in0[i], p.in1[i], p.act);
}

// grad_bias[i] += sum_r gaa[r*n + i], rows ascending exactly like
// cpuAccumulateBias (src/backend.zig:706-713): one thread per column, so the
// result is bit-identical to the reference.  Loads are coalesced across the
// threads of a row and issued eight rows ahead of the (sequential) adds.
extern "C" __global__ __launch_bounds__(256) void zn_accumulate_bias(ZnEltArgs p) {
    const int64_t col = gtid();
    if (col >= p.n) return;
    float s = p.out[col];
    const float *src = p.in0 + col;
    int64_t r = 0;
    for (; r + 8 <= p.rows; r += 8) {
        float v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = src[(r + q) * p.n];
#pragma unroll
        for (int q = 0; q < 8; ++q) s = s + v[q];
    }
    for (; r < p.rows; ++r) s = s + src[r * p.n];
    p.out[col] = s;
}

// Dense.backward's first two steps in one pass (src/layer.zig:429-445,
// 458-462): gaa = activationBackward(y, grad_out) elementwise (as
// zn_activation_backward) and, for the bias gradient, column sums of gaa
// over the rows of split blockIdx.y (rows ascending within the split).  One
// thread per column, 256 columns per workgroup, so row loads are coalesced.
extern "C" __global__ __launch_bounds__(256) void zn_dense_grad_prologue(ZnDenseGradArgs p) {
    const int64_t col = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (col >= p.n) return;
    const int64_t r0 = (int64_t)blockIdx.y * p.rows_per_split;
    const int64_t r1 = r0 + p.rows_per_split < p.rows ? r0 + p.rows_per_split : p.rows;
    float s = 0.0f;
    int64_t r = r0;
    for (; r + 4 <= r1; r += 4) {
        float y[4], g[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            y[q] = p.y[(r + q) * p.n + col];
            g[q] = p.go[(r + q) * p.n + col];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float d = zn_act_backward(y[q], g[q], p.act);
            if (p.gaa) p.gaa[(r + q) * p.n + col] = d;
            s = s + d;
        }
    }
    for (; r < r1; ++r) {
        const float d = zn_act_backward(p.y[r * p.n + col], p.go[r * p.n + col], p.act);
        if (p.gaa) p.gaa[r * p.n + col] = d;
        s = s + d;
    }
    p.partial[(int64_t)blockIdx.y * p.n + col] = s;
}

// Filter tap index <-> (ic, kh, kw) for the two col K orders.
__device__ __forceinline__ void zn_tap_decode(const ZnIm2colArgs &p, int tap, int &ic, int &kh, int &kw) {
    if (p.k_order == 0) {
        const int kpos = tap / p.channels;
        ic = tap - kpos * p.channels;
        kh = kpos / p.k_w;
        kw = kpos - kh * p.k_w;
    } else {
        const int khw = p.k_h * p.k_w;
        ic = tap / khw;
        const int kpos = tap - ic * khw;
        kh = kpos / p.k_w;
        kw = kpos - kh * p.k_w;
    }
}

// Backend.im2col (src/backend.zig:3775-3827): col[(b*OH*OW + oh*OW + ow)][tap],
// zero outside the padded input.  A workgroup fills a tile of 64 col rows x
// 64 taps: lanes run along the rows (neighbouring output pixels, so the NCHW
// reads are contiguous) into LDS, then along the taps for the col stores.
constexpr int kIm2colTile = 64;
extern "C" __global__ __launch_bounds__(256) void zn_im2col(ZnIm2colArgs p) {
    __shared__ float tile[kIm2colTile][kIm2colTile + 1];
    const int kc = p.k_h * p.k_w * p.channels;
    const int hw = p.out_h * p.out_w;
    const int64_t rows = (int64_t)p.batch * hw;
    const int64_t row_tiles = (rows + kIm2colTile - 1) / kIm2colTile;
    const int tap_tiles = (kc + kIm2colTile - 1) / kIm2colTile;
    const int64_t units = row_tiles * tap_tiles;
    const int lane = threadIdx.x & 63, sub = threadIdx.x >> 6;
    for (int64_t u = blockIdx.x; u < units; u += gridDim.x) {
        const int64_t row0 = (u / tap_tiles) * kIm2colTile;
        const int tap0 = (int)(u % tap_tiles) * kIm2colTile;
        // gather: this lane's row (output pixel) is fixed, its taps step by 4
        const int64_t row = row0 + lane;
        const int64_t b = row / hw;
        const int r = (int)(row - b * hw);
        const int oh = r / p.out_w, ow = r - oh * p.out_w;
        const float *img = p.image + b * p.channels * (int64_t)p.in_h * p.in_w;
        for (int t = sub; t < kIm2colTile; t += 4) {
            const int tap = tap0 + t;
            float v = 0.0f;
            if (row < rows && tap < kc) {
                int ic, kh, kw;
                zn_tap_decode(p, tap, ic, kh, kw);
                const int ih = oh * p.stride_h - p.pad_h + kh;
                const int iw = ow * p.stride_w - p.pad_w + kw;
                if (ih >= 0 && iw >= 0 && ih < p.in_h && iw < p.in_w)
                    v = img[((int64_t)ic * p.in_h + ih) * p.in_w + iw];
            }
            tile[t][lane] = v;
        }
        __syncthreads();
        for (int rr = sub; rr < kIm2colTile; rr += 4) {
            const int64_t orow = row0 + rr;
            const int tap = tap0 + lane;
            if (orow < rows && tap < kc) p.col[orow * kc + tap] = tile[lane][rr];
        }
        __syncthreads();  // the tile is rewritten by the next unit
    }
}

// Backend.col2im (src/backend.zig:3833-3877) as a gather: every NCHW output
// element is the sum, from 0, of the col entries that land on it in the
// reference's order (output rows oh, then ow, ascending; each (oh, ow)
// reaches a given input pixel through at most one tap), so the result is
// bit-identical to the reference's scatter.  A workgroup owns kCol2imW
// pixels of one input row for 64 channels at a time: lanes run along the
// channel (contiguous in the im2col-order col rows) while summing, and the
// sums go through LDS so the NCHW stores run along the row.
constexpr int kCol2imW = 64;
extern "C" __global__ __launch_bounds__(256) void zn_col2im(ZnIm2colArgs p) {
    __shared__ float tile[64][kCol2imW + 1];
    const int kc = p.k_h * p.k_w * p.channels;
    const int64_t hw = (int64_t)p.out_h * p.out_w;
    const int wtiles = (p.in_w + kCol2imW - 1) / kCol2imW;
    const int64_t units = (int64_t)p.batch * p.in_h * wtiles;
    const int lane_c = threadIdx.x & 63, sub = threadIdx.x >> 6;  // channel in group, pixel phase (0..3)
    for (int64_t u = blockIdx.x; u < units; u += gridDim.x) {
        const int wt = (int)(u % wtiles);
        const int64_t bh = u / wtiles;
        const int ih = (int)(bh % p.in_h);
        const int64_t b = bh / p.in_h;
        const int iw0 = wt * kCol2imW;
        const int hh = ih + p.pad_h;
        const int oh_lo = hh >= p.k_h ? (hh - p.k_h) / p.stride_h + 1 : 0;
        const int oh_hi = min(hh / p.stride_h, p.out_h - 1);
        const float *cb = p.col + b * hw * kc;
        for (int c0 = 0; c0 < p.channels; c0 += 64) {
            const int ic = c0 + lane_c;
            for (int x = sub; x < kCol2imW; x += 4) {
                const int iw = iw0 + x;
                float sum = 0.0f;
                if (ic < p.channels && iw < p.in_w) {
                    const int ww = iw + p.pad_w;
                    const int ow_lo = ww >= p.k_w ? (ww - p.k_w) / p.stride_w + 1 : 0;
                    const int ow_hi = min(ww / p.stride_w, p.out_w - 1);
                    for (int oh = oh_lo; oh <= oh_hi; ++oh) {
                        const int kh = hh - oh * p.stride_h;
                        for (int ow = ow_lo; ow <= ow_hi; ++ow) {
                            const int kw = ww - ow * p.stride_w;
                            const int tap =
                                p.k_order == 0 ? (kh * p.k_w + kw) * p.channels + ic : (ic * p.k_h + kh) * p.k_w + kw;
                            sum = sum + cb[((int64_t)oh * p.out_w + ow) * kc + tap];
                        }
                    }
                }
                tile[lane_c][x] = sum;
            }
            __syncthreads();
            for (int cc = sub; cc < 64; cc += 4) {
                const int c = c0 + cc;
                const int iw = iw0 + lane_c;
                if (c < p.channels && iw < p.in_w)
                    p.image[((b * p.channels + c) * p.in_h + ih) * (int64_t)p.in_w + iw] = tile[cc][lane_c];
            }
            __syncthreads();  // the tile is rewritten for the next channel group
        }
    }
}

// Row sums: out[r] = sum of in[r*n .. r*n + n), one workgroup per row, each
// thread a fixed strided subset in ascending order, then a fixed tree, so
// results do not depend on scheduling.  The per-(image, channel) stage of
// the conv grad_bias (src/backend.zig:3073-3074, 3983-3993).  Rows of whole
// float4s (16-byte aligned) are read 16 bytes at a time, each of a thread's
// four lanes summed apart and the four added at the end: C5's 4096 rows of
// 3136 went from 11.9 to 10.3 us on MI355X.
extern "C" __global__ __launch_bounds__(256) void zn_row_sum(ZnEltArgs p) {
    __shared__ float red[256];
    const bool vec = (p.n & 3) == 0 && (reinterpret_cast<uintptr_t>(p.in0) & 15) == 0;
    for (int64_t r = blockIdx.x; r < p.rows; r += gridDim.x) {
        const float *src = p.in0 + r * p.n;
        float s = 0.0f;
        if (vec) {
            const zn_f32x4 *src4 = reinterpret_cast<const zn_f32x4 *>(src);
            zn_f32x4 a = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
            for (int64_t i = threadIdx.x; i < (p.n >> 2); i += 256) a = a + src4[i];
            s = (a[0] + a[1]) + (a[2] + a[3]);
        } else {
            for (int64_t i = threadIdx.x; i < p.n; i += 256) s = s + src[i];
        }
        __syncthreads();  // `red` may still be read for the previous row
        red[threadIdx.x] = s;
        __syncthreads();
        for (int w = 128; w > 0; w >>= 1) {
            if ((int)threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
            __syncthreads();
        }
        if (threadIdx.x == 0) p.out[r] = red[0];
    }
}

// A GEMM operand whose rows are not 16-byte aligned (or not whole float4s)
// copied into rows of ld_dst floats with a zero tail, so the GEMM can stage
// it with 16-byte loads.  A copy (bit-exact); one float4 of dst per thread
// and step.
extern "C" __global__ __launch_bounds__(256) void zn_pack_rows(ZnPack2Args a) {
    const ZnPackArgs &p = a.op[blockIdx.y];  // both GEMM operands in one launch (gridDim.y <= 2)
    const int64_t per_row = p.ld_dst >> 2;
    const int64_t total = p.rows * per_row;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / per_row, c = (i - r * per_row) * 4;
        const float *src = p.src + r * p.ld_src;
        zn_f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = c + e < p.cols ? src[c + e] : 0.0f;
        reinterpret_cast<zn_f32x4 *>(p.dst)[i] = v;
    }
}

// NCHW -> NHWC for the convolution forward's 4-channel gather: 32x32 tiles
// through LDS, read along pixels and written along channels (both
// coalesced).  A permutation (bit-exact).  Grid-stride over (image, tile).
extern "C" __global__ __launch_bounds__(256) void zn_nchw_to_nhwc(ZnTransposeArgs p) {
    __shared__ float tile[32][33];
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    const int64_t tc = (p.channels + 31) / 32, tp = (p.pixels + 31) / 32;
    const int64_t per_image = tc * tp, total = per_image * p.batch;
    // whole float4s on both sides: one 16-byte load (4 pixels of a channel)
    // and one 16-byte store (4 channels of a pixel) per thread and tile
    // (C5's 32 x 64 x 56 x 56 batch on MI355X: 11.8 -> 9.6 us)
    const bool vec = (p.pixels & 3) == 0 && (p.channels & 3) == 0 &&
                     ((reinterpret_cast<uintptr_t>(p.src) | reinterpret_cast<uintptr_t>(p.dst)) & 15) == 0;
    const int g8 = threadIdx.x >> 3, l8 = threadIdx.x & 7;  // 32 x 8 groups of 4
    for (int64_t t = blockIdx.x; t < total; t += gridDim.x) {
        const int64_t b = t / per_image, r = t - b * per_image;
        const int64_t c0 = (r / tp) * 32, p0 = (r % tp) * 32;
        const float *src = p.src + b * p.channels * p.pixels;
        float *dst = p.dst + b * p.channels * p.pixels;
        __syncthreads();  // the previous tile's reads of `tile` are done
        if (vec) {
            {
                const int64_t c = c0 + g8, q = p0 + 4 * l8;  // 4 pixels of channel c
                if (c < p.channels && q < p.pixels) {
                    const zn_f32x4 v = *reinterpret_cast<const zn_f32x4 *>(src + c * p.pixels + q);
#pragma unroll
                    for (int e = 0; e < 4; ++e) tile[g8][4 * l8 + e] = v[e];
                }
            }
            __syncthreads();
            {
                const int64_t q = p0 + g8, c = c0 + 4 * l8;  // 4 channels of pixel q
                if (c < p.channels && q < p.pixels) {
                    zn_f32x4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = tile[4 * l8 + e][g8];
                    *reinterpret_cast<zn_f32x4 *>(dst + q * p.channels + c) = v;
                }
            }
            continue;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t c = c0 + ty + 8 * i, q = p0 + tx;
            if (c < p.channels && q < p.pixels) tile[ty + 8 * i][tx] = src[c * p.pixels + q];
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t q = p0 + ty + 8 * i, c = c0 + tx;
            if (c < p.channels && q < p.pixels) dst[q * p.channels + c] = tile[tx][ty + 8 * i];
        }
    }
}

// W' for the stride-1 transposed-convolution GEMM of the input gradient
// (cpuConv2dBackwardIm2col's grad_col = go2 . W followed by col2im, src/
// backend.zig:3995-4060, as one GEMM): the [OC][kH*kW][C] weights regrouped
// to [C][kH*kW][OC].  A pure permutation (bit-exact); weights are small, so
// one thread per output element with coalesced writes is enough.
extern "C" __global__ __launch_bounds__(256) void zn_weight_regroup(ZnRegroupArgs p) {
    const int64_t per_ic = (int64_t)p.taps_per_channel * p.out_channels;
    const int64_t total = per_ic * p.channels;
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < total; o += (int64_t)gridDim.x * 256) {
        const int64_t ic = o / per_ic, r = o - ic * per_ic;
        const int64_t t = r / p.out_channels, oc = r - t * p.out_channels;
        p.out[o] = p.in[(oc * p.taps_per_channel + t) * p.channels + ic];
    }
}

namespace {

constexpr int kSoftmaxThreads = 256;
constexpr int kSoftmaxPerThread = 8;  // rows up to 2048 stay in registers

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Block-wide reduction of one value per thread (max or sum).
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float *red) {
    v = MAX ? wave_max(v) : wave_sum(v);
    const int wave = threadIdx.x / 64, lane = threadIdx.x & 63;
    __syncthreads();  // `red` may still be read from the previous reduction
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < kSoftmaxThreads / 64; ++w) r = MAX ? fmaxf(r, red[w]) : r + red[w];
    return r;
}

}  // namespace

// Row softmax of scaled scores, in place allowed (out may equal in0):
// out[r, :] = exp(s - max) / sum(exp(s - max)) with s = in0[r, :] * value,
// the steps of cpuAttentionForward (src/backend.zig:3201-3214).  One
// workgroup per row; rows up to 2048 are read once and kept in registers.
extern "C" __global__ __launch_bounds__(256) void zn_softmax_rows(ZnEltArgs p) {
    __shared__ float red[kSoftmaxThreads / 64];
    const float scale = p.value;
    for (int64_t r = blockIdx.x; r < p.rows; r += gridDim.x) {
        const float *src = p.in0 + r * p.n;
        float *dst = p.out + r * p.n;
        if (p.n <= kSoftmaxThreads * kSoftmaxPerThread) {
            float v[kSoftmaxPerThread];
            float mx = -INFINITY;
#pragma unroll
            for (int q = 0; q < kSoftmaxPerThread; ++q) {
                const int64_t i = threadIdx.x + (int64_t)q * kSoftmaxThreads;
                v[q] = i < p.n ? src[i] * scale : -INFINITY;
                mx = fmaxf(mx, v[q]);
            }
            mx = block_reduce<true>(mx, red);
            float sum = 0.0f;
#pragma unroll
            for (int q = 0; q < kSoftmaxPerThread; ++q) {
                const int64_t i = threadIdx.x + (int64_t)q * kSoftmaxThreads;
                v[q] = i < p.n ? expf(v[q] - mx) : 0.0f;
                sum += v[q];
            }
            sum = block_reduce<false>(sum, red);
#pragma unroll
            for (int q = 0; q < kSoftmaxPerThread; ++q) {
                const int64_t i = threadIdx.x + (int64_t)q * kSoftmaxThreads;
                if (i < p.n) dst[i] = v[q] / sum;
            }
        } else {
            float mx = -INFINITY;
            for (int64_t i = threadIdx.x; i < p.n; i += kSoftmaxThreads) mx = fmaxf(mx, src[i] * scale);
            mx = block_reduce<true>(mx, red);
            float sum = 0.0f;
            for (int64_t i = threadIdx.x; i < p.n; i += kSoftmaxThreads) {
                const float e = expf(src[i] * scale - mx);
                dst[i] = e;
                sum += e;
            }
            sum = block_reduce<false>(sum, red);
            for (int64_t i = threadIdx.x; i < p.n; i += kSoftmaxThreads) dst[i] = dst[i] / sum;
        }
    }
}

// One wave that returns after p.value microseconds (read from the 100 MHz
// constant clock, s_memrealtime), sleeping in between.  It keeps a stream
// busy while the host queues the launches that follow it, so that those run
// back to back from the queue and their timing measures the device, not the
// rate at which the host submits (the "blocking kernel" of GPU benchmark
// harnesses).  At most p.n sleeps: the wait ends even if the clock stalls.
extern "C" __global__ __launch_bounds__(64) void zn_hold_stream(ZnEltArgs p) {
    const uint64_t start = __builtin_amdgcn_s_memrealtime();
    const uint64_t ticks = (uint64_t)(p.value * 100.0f);
    for (int64_t i = 0; i < p.n; ++i) {
        __builtin_amdgcn_s_sleep(8);
        if (__builtin_amdgcn_s_memrealtime() - start >= ticks) break;
    }
}
