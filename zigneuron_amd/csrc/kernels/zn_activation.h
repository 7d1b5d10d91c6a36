// Activation derivative shared by the elementwise kernels and the GEMM
// epilogues that apply it: grad_in = grad_out * act'(y), from the activated
// output y as the reference does (src/optimization.zig:229-303).  The same
// expression everywhere, so every kernel that computes it rounds alike.
#ifndef ZN_ACTIVATION_H
#define ZN_ACTIVATION_H

#include <hip/hip_runtime.h>

__device__ __forceinline__ float zn_act_backward(float y, float go, int act) {
    switch (act) {
    case 1: return y > 0.0f ? go : 0.0f;
    case 2: return (go * y) * (1.0f - y);
    case 3: return go * (1.0f - y * y);
    default: return go;
    }
}

#endif
