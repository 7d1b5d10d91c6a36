// Elementwise and reduction helpers of the Dense path for gfx950:
// fill, copy (also the HBM reference kernel for counter calibration), bias
// add, activation forward/backward and the bias-gradient column sum.
// All are HBM-bound streaming kernels: coalesced, grid-stride, 16-byte
// accesses where alignment allows.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../zn_kernel_args.h"

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

// Activation backward from the activated output y (src/optimization.zig:229-303).
__device__ __forceinline__ float act_backward(float y, float go, int act) {
    switch (act) {
    case 1: return y > 0.0f ? go : 0.0f;
    case 2: return (go * y) * (1.0f - y);
    case 3: return go * (1.0f - y * y);
    default: return go;
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
    for (int64_t i = gtid(); i < total; i += gstride()) p.out[i] = act_backward(p.in0[i], p.in1[i], p.act);
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

// Backend.im2col (src/backend.zig:3775-3827): one thread per element of
// col[(b*OH*OW + oh*OW + ow)][tap]; zero outside the padded input.  Writes
// are coalesced along the col row.
extern "C" __global__ __launch_bounds__(256) void zn_im2col(ZnIm2colArgs p) {
    const int64_t kc = (int64_t)p.k_h * p.k_w * p.channels;
    const int64_t hw = (int64_t)p.out_h * p.out_w;
    const int64_t total = (int64_t)p.batch * hw * kc;
    for (int64_t i = gtid(); i < total; i += gstride()) {
        const int64_t row = i / kc;
        int ic, kh, kw;
        zn_tap_decode(p, (int)(i - row * kc), ic, kh, kw);
        const int64_t b = row / hw;
        const int r = (int)(row - b * hw);
        const int oh = r / p.out_w, ow = r - oh * p.out_w;
        const int ih = oh * p.stride_h - p.pad_h + kh;
        const int iw = ow * p.stride_w - p.pad_w + kw;
        float v = 0.0f;
        if (ih >= 0 && iw >= 0 && ih < p.in_h && iw < p.in_w)
            v = p.image[((b * p.channels + ic) * p.in_h + ih) * (int64_t)p.in_w + iw];
        p.col[i] = v;
    }
}

// Backend.col2im (src/backend.zig:3833-3877) as a gather: one thread per
// NCHW output element, summing, from 0, the col entries that land on it in
// the reference's order (output rows oh, then ow, ascending; each (oh, ow)
// reaches a given input pixel through at most one tap), so the result is
// bit-identical to the reference's scatter.
extern "C" __global__ __launch_bounds__(256) void zn_col2im(ZnIm2colArgs p) {
    const int64_t kc = (int64_t)p.k_h * p.k_w * p.channels;
    const int64_t hw = (int64_t)p.out_h * p.out_w;
    const int64_t plane = (int64_t)p.in_h * p.in_w;
    const int64_t total = (int64_t)p.batch * p.channels * plane;
    for (int64_t i = gtid(); i < total; i += gstride()) {
        const int64_t bc = i / plane;
        const int pix = (int)(i - bc * plane);
        const int64_t b = bc / p.channels;
        const int ic = (int)(bc - b * p.channels);
        const int ih = pix / p.in_w, iw = pix - ih * p.in_w;
        // output rows whose window covers ih: 0 <= ih + pad_h - oh*stride_h < k_h
        const int hh = ih + p.pad_h, ww = iw + p.pad_w;
        const int oh_lo = hh >= p.k_h ? (hh - p.k_h) / p.stride_h + 1 : 0;
        const int oh_hi = min(hh / p.stride_h, p.out_h - 1);
        const int ow_lo = ww >= p.k_w ? (ww - p.k_w) / p.stride_w + 1 : 0;
        const int ow_hi = min(ww / p.stride_w, p.out_w - 1);
        const float *cb = p.col + b * hw * kc;
        float sum = 0.0f;
        for (int oh = oh_lo; oh <= oh_hi; ++oh) {
            const int kh = hh - oh * p.stride_h;
            for (int ow = ow_lo; ow <= ow_hi; ++ow) {
                const int kw = ww - ow * p.stride_w;
                const int tap = p.k_order == 0 ? (kh * p.k_w + kw) * p.channels + ic : (ic * p.k_h + kh) * p.k_w + kw;
                sum = sum + cb[((int64_t)oh * p.out_w + ow) * kc + tap];
            }
        }
        p.image[i] = sum;
    }
}

// out[c] = sum over (b, p) of in[(b*C + c)*hw + p]: one workgroup per
// channel, each thread a fixed strided subset in ascending order, then a
// fixed tree, so results do not depend on scheduling (the grad_bias of
// cpuConv2dBackward, src/backend.zig:3073-3074, 3983-3993).
extern "C" __global__ __launch_bounds__(256) void zn_channel_sum(ZnChannelSumArgs p) {
    __shared__ float red[256];
    for (int64_t c = blockIdx.x; c < p.channels; c += gridDim.x) {
        float s = 0.0f;
        for (int64_t b = 0; b < p.batch; ++b) {
            const float *src = p.in + (b * p.channels + c) * p.hw;
            for (int64_t i = threadIdx.x; i < p.hw; i += 256) s = s + src[i];
        }
        __syncthreads();  // `red` may still be read for the previous channel
        red[threadIdx.x] = s;
        __syncthreads();
        for (int w = 128; w > 0; w >>= 1) {
            if ((int)threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
            __syncthreads();
        }
        if (threadIdx.x == 0) p.out[c] = red[0];
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
