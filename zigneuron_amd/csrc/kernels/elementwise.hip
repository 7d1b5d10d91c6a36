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
