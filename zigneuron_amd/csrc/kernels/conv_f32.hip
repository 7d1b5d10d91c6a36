// Exported implicit-GEMM convolution kernels for gfx950 (forward, input and
// weight gradients), on the GEMM core of gemm_core.h with gathered B operands.
// The 64x64 kernels of the three gathers that load only by DMA (transposed,
// NHWC forward, NHWC weight gradient) run the pinned three-stage loop at
// BK 16 (24 KB of LDS, six workgroups per CU): on MI355X, C5 forward
// 160.3 -> 156.6 us, a 4 x 128 x 14 x 14 -> 256 convolution 21.9 -> 19.8 us
// forward and 50.6 -> 46.5 us backward, bit-identical results.  The host's
// K granularity for the 64x64 tile (32: split-K chunks, the NHWC forward's
// one-tap slices) is a multiple of that BK.
#include "gemm_core.h"

// Implicit-GEMM convolution, per image b = blockIdx.y:
// out_b[OC][OH*OW] = W[OC][K] . im2col(input_b)^T (+ bias[oc]), an NN GEMM
// whose B operand is gathered from the NCHW input (ZnConvGeom).  _v: W rows
// are 16-byte aligned; _g: the input is gathered in chunks of 4 pixels with
// 16-byte loads (stride_w == 1, out_w % 4 == 0), otherwise element by element.
#define ZN_CONV_KERNEL(TILE, BM, BN, BK, WM, WN, MINB, WA, G, SUFFIX)                             \
    extern "C" __global__ __launch_bounds__(WM *WN * 64, MINB) void zn_conv_nn_##TILE##SUFFIX(ZnGemmArgs p) { \
        gemm_tile_dma<BM, BN, BK, WM, WN, true, false, WA, 4, G>(p);                              \
    }
#define ZN_CONV_TILE(TILE, BM, BN, BK, WM, WN, MINB)                                              \
    ZN_CONV_KERNEL(TILE, BM, BN, BK, WM, WN, MINB, 16, kGIm2col, _v)                             \
    ZN_CONV_KERNEL(TILE, BM, BN, BK, WM, WN, MINB, 4, kGIm2col, )                                \
    ZN_CONV_KERNEL(TILE, BM, BN, BK, WM, WN, MINB, 16, kGIm2col4, _v_g)                          \
    ZN_CONV_KERNEL(TILE, BM, BN, BK, WM, WN, MINB, 4, kGIm2col4, _g)

ZN_CONV_TILE(x, 256, 128, 16, 4, 2, 1)
ZN_CONV_TILE(l, 128, 128, 16, 2, 2, 4)
ZN_CONV_TILE(n, 128, 64, 16, 2, 1, 1)
ZN_CONV_TILE(m, 64, 64, 32, 2, 2, 1)
ZN_CONV_TILE(s, 32, 32, 32, 1, 1, 1)

// Input gradient of a stride-1 convolution, per image b = blockIdx.y:
// grad_input_b[C][H*W] = W'[C][K] . B^T, NT, W' = weights regrouped as
// [ic][(kh*kW + kw)*OC + oc] and B gathered from grad_output rows
// (ConvTGatherStage).  _v: W' rows are 16-byte aligned.
#define ZN_CONVT_KERNEL(TILE, LOOP, BM, BN, BK, WM, WN, MINB, WA, SUFFIX)                       \
    extern "C" __global__ __launch_bounds__(WM *WN * 64, MINB) void zn_convt_nt_##TILE##SUFFIX(ZnGemmArgs p) { \
        LOOP<BM, BN, BK, WM, WN, true, true, WA, 16, kGTransposed>(p); \
    }
#define ZN_CONVT_TILE(TILE, LOOP, BM, BN, BK, WM, WN, MINB) \
    ZN_CONVT_KERNEL(TILE, LOOP, BM, BN, BK, WM, WN, MINB, 16, _v) \
    ZN_CONVT_KERNEL(TILE, LOOP, BM, BN, BK, WM, WN, MINB, 4, )

ZN_CONVT_TILE(x, gemm_tile_dma, 256, 128, 16, 4, 2, 1)
ZN_CONVT_TILE(l, gemm_tile_dma, 128, 128, 16, 2, 2, 4)
ZN_CONVT_TILE(n, gemm_tile_dma, 128, 64, 16, 2, 1, 1)
ZN_CONVT_TILE(m, gemm_tile_pinned, 64, 64, 16, 2, 2, 2)
ZN_CONVT_TILE(s, gemm_tile_dma, 32, 32, 32, 1, 1, 1)

// Weight gradient of a convolution with stride_w == 1 and out_w % 4 == 0:
// grad_W[OC][taps] = go2^T . col with K = the output pixels of all images,
// A = grad_output read as [pixels][OC] rows (X-contiguous, like TN) and
// B = col gathered from the NCHW input (ConvWGatherStage).  _v: OC % 4 == 0
// and grad_output 16-byte aligned.
#define ZN_CONVW_KERNEL(TILE, BM, BN, BK, WM, WN, MINB, WA, SUFFIX)                                \
    extern "C" __global__ __launch_bounds__(WM *WN * 64, MINB) void zn_convw_tn_##TILE##SUFFIX(ZnGemmArgs p) { \
        gemm_tile_dma<BM, BN, BK, WM, WN, false, true, WA, 16, kGWeight>(p);                     \
    }
#define ZN_CONVW_TILE(TILE, BM, BN, BK, WM, WN, MINB)                                              \
    ZN_CONVW_KERNEL(TILE, BM, BN, BK, WM, WN, MINB, 16, _v)                                       \
    ZN_CONVW_KERNEL(TILE, BM, BN, BK, WM, WN, MINB, 4, )

ZN_CONVW_TILE(x, 256, 128, 16, 4, 2, 1)
ZN_CONVW_TILE(l, 128, 128, 16, 2, 2, 4)
ZN_CONVW_TILE(n, 128, 64, 16, 2, 1, 1)
ZN_CONVW_TILE(m, 64, 64, 32, 2, 2, 1)
ZN_CONVW_TILE(s, 32, 32, 32, 1, 1, 1)

// Convolution forward on an NHWC copy of the input, per image b = blockIdx.y:
// out_b[OC][OH*OW] = W[OC][K] . B^T (+ bias[oc]), NT, W in the im2col K order
// and B gathered 4 channels at a time (ConvNhwcGatherStage, C % 4 == 0, any
// stride).  _v: W rows are 16-byte aligned.
#define ZN_CONVF_KERNEL(TILE, LOOP, BM, BN, BK, WM, WN, MINB, WA, SUFFIX)                       \
    extern "C" __global__ __launch_bounds__(WM *WN * 64, MINB) void zn_convf_nt_##TILE##SUFFIX(ZnGemmArgs p) { \
        LOOP<BM, BN, BK, WM, WN, true, true, WA, 16, kGNhwc>(p); \
    }
#define ZN_CONVF_TILE(TILE, LOOP, BM, BN, BK, WM, WN, MINB) \
    ZN_CONVF_KERNEL(TILE, LOOP, BM, BN, BK, WM, WN, MINB, 16, _v) \
    ZN_CONVF_KERNEL(TILE, LOOP, BM, BN, BK, WM, WN, MINB, 4, )

ZN_CONVF_TILE(x, gemm_tile_dma, 256, 128, 16, 4, 2, 1)
ZN_CONVF_TILE(l, gemm_tile_dma, 128, 128, 16, 2, 2, 4)
ZN_CONVF_TILE(n, gemm_tile_dma, 128, 64, 16, 2, 1, 1)
ZN_CONVF_TILE(m, gemm_tile_pinned, 64, 64, 16, 2, 2, 2)
ZN_CONVF_TILE(s, gemm_tile_dma, 32, 32, 32, 1, 1, 1)

// Weight gradient from an NHWC copy of the input: grad_W[OC][taps] =
// go2^T . col, TN, K = the output pixels of all images, B gathered 4 channels
// at a time (ConvNhwcWGatherStage, C % 4 == 0, any stride).  _v: OC % 4 == 0
// and grad_output 16-byte aligned.
#define ZN_CONVWN_KERNEL(TILE, LOOP, BM, BN, BK, WM, WN, MINB, WA, SUFFIX)                      \
    extern "C" __global__ __launch_bounds__(WM *WN * 64, MINB) void zn_convwn_tn_##TILE##SUFFIX(ZnGemmArgs p) { \
        LOOP<BM, BN, BK, WM, WN, false, false, WA, 16, kGNhwcW>(p); \
    }
#define ZN_CONVWN_TILE(TILE, LOOP, BM, BN, BK, WM, WN, MINB) \
    ZN_CONVWN_KERNEL(TILE, LOOP, BM, BN, BK, WM, WN, MINB, 16, _v) \
    ZN_CONVWN_KERNEL(TILE, LOOP, BM, BN, BK, WM, WN, MINB, 4, )

ZN_CONVWN_TILE(x, gemm_tile_dma, 256, 128, 16, 4, 2, 1)
ZN_CONVWN_TILE(l, gemm_tile_dma, 128, 128, 16, 2, 2, 4)
ZN_CONVWN_TILE(n, gemm_tile_dma, 128, 64, 16, 2, 1, 1)
ZN_CONVWN_TILE(m, gemm_tile_pinned, 64, 64, 16, 2, 2, 2)
// 128x128 on the register-staged loop (16-byte grad_output rows only): one
// round of tiles x K slices
extern "C" __global__ __launch_bounds__(512, 1) void zn_convwn_tn_r_v(ZnGemmArgs p) {
    gemm_tile_wide<128, 128, 16, 2, 4, false, false, kGNhwcW>(p);
}
ZN_CONVWN_TILE(s, gemm_tile_dma, 32, 32, 32, 1, 1, 1)
