// Exported fp32 GEMM kernels for gfx950: the plain, persistent and
// intra-workgroup split-K GEMMs, the split-K reduce and the grouped Dense
// backward launches (device code in gemm_core.h).
#include "gemm_core.h"

// Exported kernels: zn_sgemm_<layout>_<tile>[_v].  Layout letters follow
// the reference: nn = Backend.matMul, nt = matMulTransposeB, tn =
// matMulTransposeA.  Tiles (macro tile, waves x wave tile, main loop):
//   x = 256x128, 8 waves of 64x64    large problems (two workgroups per CU)
//   l = 128x128, 4 waves of 64x64
//   n = 128x64,  2 waves of 64x64    narrow N (attention P.V, N = 64)
//   m = 64x64,   4 waves of 32x32    mid-size problems (BK 32, pinned loop)
//   s = 32x32,   1 wave              small problems (BK 32)
//   r = 128x128, 8 waves             one round of tiles, one workgroup per
//                                    CU (16-byte rows: 64x32 wave tiles,
//                                    BK 16, gemm_tile_wide; 4-byte rows:
//                                    32x64, BK 32, pinned loop)
//   h = 64x64,   4 waves of 32x32    several rounds (BK 16, pinned loop,
//                                    six workgroups per CU)
//   w = 256x256, 8 waves of 128x64   full rounds of large problems (BK 16,
//                                    gemm_tile_wide, one workgroup per CU;
//                                    16-byte loads staged through registers,
//                                    no plain variant)
// x, l, n and s run gemm_tile_dma's two-stage loop, m, h and the plain r
// gemm_tile_pinned's three-stage one, w and the 16-byte r gemm_tile_wide.
// The _v variants load operands 16 bytes at a time (aligned rows, contiguous
// extents a multiple of 4): straight into LDS, or through registers on
// gemm_tile_wide; the plain ones 4 bytes at a time straight into LDS.
#define ZN_GEMM_KERNEL(NAME, LOOP, BM, BN, BK, WM, WN, AK, BKC, VEC, MINB)                      \
    extern "C" __global__ __launch_bounds__(WM *WN * 64, MINB) void NAME(ZnGemmArgs p) {        \
        LOOP<BM, BN, BK, WM, WN, AK, BKC, (VEC) ? 16 : 4, (VEC) ? 16 : 4>(p);                    \
    }

#define ZN_GEMM_LAYOUTS(TILE, LOOP, BM, BN, BK, WM, WN, MINB, VEC, SUFFIX)                      \
    ZN_GEMM_KERNEL(zn_sgemm_nn_##TILE##SUFFIX, LOOP, BM, BN, BK, WM, WN, true, false, VEC, MINB) \
    ZN_GEMM_KERNEL(zn_sgemm_nt_##TILE##SUFFIX, LOOP, BM, BN, BK, WM, WN, true, true, VEC, MINB)  \
    ZN_GEMM_KERNEL(zn_sgemm_tn_##TILE##SUFFIX, LOOP, BM, BN, BK, WM, WN, false, false, VEC, MINB)

#define ZN_GEMM_TILE(TILE, LOOP, BM, BN, BK, WM, WN, MINB)                                      \
    ZN_GEMM_LAYOUTS(TILE, LOOP, BM, BN, BK, WM, WN, MINB, true, _v)                              \
    ZN_GEMM_LAYOUTS(TILE, LOOP, BM, BN, BK, WM, WN, MINB, false, )

ZN_GEMM_TILE(x, gemm_tile_dma, 256, 128, 16, 4, 2, 1)
ZN_GEMM_TILE(l, gemm_tile_dma, 128, 128, 16, 2, 2, 4)
ZN_GEMM_TILE(n, gemm_tile_dma, 128, 64, 16, 2, 1, 1)
ZN_GEMM_TILE(m, gemm_tile_pinned, 64, 64, 32, 2, 2, 1)
ZN_GEMM_TILE(s, gemm_tile_dma, 32, 32, 32, 1, 1, 1)
// r: 16-byte rows on gemm_tile_wide (8 waves of 64x32, BK 16, operands
// staged through registers), 4-byte rows on gemm_tile_pinned (8 waves of
// 32x64, BK 32); both keep the K order of the other tiles
ZN_GEMM_LAYOUTS(r, gemm_tile_pinned, 128, 128, 32, 4, 2, 1, false, )
#define ZN_GEMM_R_WIDE(LAYOUT, AK, BKC)                                                          \
    extern "C" __global__ __launch_bounds__(512, 1) void zn_sgemm_##LAYOUT##_r_v(ZnGemmArgs p) { \
        gemm_tile_wide<128, 128, 16, 2, 4, AK, BKC>(p);                                          \
    }
ZN_GEMM_R_WIDE(nn, true, false)
ZN_GEMM_R_WIDE(nt, true, true)
ZN_GEMM_R_WIDE(tn, false, false)
// zn_sgemm_<layout>_r_u: the same loop for rows that are not whole float4s,
// loaded as they lie with 16-byte loads (gemm_tile_wide's UA), instead of
// packed copies or 4-byte loads
#define ZN_GEMM_R_UNALIGNED(LAYOUT, AK, BKC)                                                     \
    extern "C" __global__ __launch_bounds__(512, 1) void zn_sgemm_##LAYOUT##_r_u(ZnGemmArgs p) { \
        gemm_tile_wide<128, 128, 16, 2, 4, AK, BKC, kGNone, true>(p);                            \
    }
ZN_GEMM_R_UNALIGNED(nn, true, false)
ZN_GEMM_R_UNALIGNED(nt, true, true)
ZN_GEMM_R_UNALIGNED(tn, false, false)
ZN_GEMM_TILE(h, gemm_tile_pinned, 64, 64, 16, 2, 2, 2)

#define ZN_GEMM_WIDE(LAYOUT, AK, BKC)                                                            \
    extern "C" __global__ __launch_bounds__(512, 1) void zn_sgemm_##LAYOUT##_w_v(ZnGemmArgs p) { \
        gemm_tile_wide<256, 256, 16, 2, 4, AK, BKC>(p);                                          \
    }
ZN_GEMM_WIDE(nn, true, false)
ZN_GEMM_WIDE(nt, true, true)
ZN_GEMM_WIDE(tn, false, false)

// Intra-workgroup split-K GEMMs (gemm_ksplit) on 32x32 tiles, BK 32, with
// KS = 4 or 8 waves: zn_sgemmk<KS>_<layout>[_v], for problems of at most one
// workgroup per CU whose tiles would otherwise need a split-K reduce launch.
// zn_sgemmk4s_<layout>[_v]: K split over workgroups as well (blockIdx.z),
// the last workgroup of each tile adding the partial tiles (p.ws,
// p.counters).
#define ZN_GEMMK_KERNEL(NAME, KS, AK, BKC, W, XS, PF)                                            \
    extern "C" __global__ __launch_bounds__(KS * 64, 1) void NAME(ZnGemmArgs p) {               \
        __shared__ __attribute__((aligned(1024))) float lds[KS * 2 * (32 + 32) * 32];            \
        switch (p.act) {                                                                         \
        case 1: gemm_ksplit<32, 32, 32, KS, AK, BKC, W, W, 1, XS, PF>(p, lds); break;            \
        case 2: gemm_ksplit<32, 32, 32, KS, AK, BKC, W, W, 2, XS, PF>(p, lds); break;            \
        case 3: gemm_ksplit<32, 32, 32, KS, AK, BKC, W, W, 3, XS, PF>(p, lds); break;            \
        default: gemm_ksplit<32, 32, 32, KS, AK, BKC, W, W, 0, XS, PF>(p, lds); break;           \
        }                                                                                        \
    }
#define ZN_GEMMK_LAYOUTS(KS, W, SUFFIX, XS, PF, S)                                              \
    ZN_GEMMK_KERNEL(zn_sgemmk##KS##S##_nn##SUFFIX, KS, true, false, W, XS, PF)                   \
    ZN_GEMMK_KERNEL(zn_sgemmk##KS##S##_nt##SUFFIX, KS, true, true, W, XS, PF)                    \
    ZN_GEMMK_KERNEL(zn_sgemmk##KS##S##_tn##SUFFIX, KS, false, false, W, XS, PF)

ZN_GEMMK_LAYOUTS(4, 16, _v, false, false, )
ZN_GEMMK_LAYOUTS(4, 4, , false, false, )
ZN_GEMMK_LAYOUTS(8, 16, _v, false, false, )
ZN_GEMMK_LAYOUTS(8, 4, , false, false, )
ZN_GEMMK_LAYOUTS(4, 16, _v, true, true, s)
ZN_GEMMK_LAYOUTS(4, 4, , true, true, s)

// The same on 16x16 tiles (gemm_ksplit16), at most one workgroup per CU:
// zn_sgemmq4_<layout>[_v] on four waves with up to 8 LDS stages each (every
// slice of a wave in flight), zn_sgemmq8_<layout>[_v] on eight waves with
// one stage each (K's slices dealt out evenly: a wave requests a slice,
// waits for it and multiplies it before requesting the next); and
// zn_sgemmq4m_<layout>[_v] on four waves with 2 stages (several workgroups
// per CU).
#define ZN_GEMMQ_KERNEL(NAME, AK, BKC, W, KS, NSMAX, MINB)                                       \
    extern "C" __global__ __launch_bounds__(KS * 64, MINB) void NAME(ZnGemmArgs p) {           \
        constexpr int kStages = NSMAX < (W == 16 ? 8 : 4) ? NSMAX : (W == 16 ? 8 : 4);           \
        __shared__ __attribute__((aligned(1024))) float lds[KS * kStages * 32 * 32];             \
        switch (p.act) {                                                                         \
        case 1: gemm_ksplit16<KS, AK, BKC, W, 1, NSMAX>(p, lds); break;                          \
        case 2: gemm_ksplit16<KS, AK, BKC, W, 2, NSMAX>(p, lds); break;                          \
        case 3: gemm_ksplit16<KS, AK, BKC, W, 3, NSMAX>(p, lds); break;                          \
        default: gemm_ksplit16<KS, AK, BKC, W, 0, NSMAX>(p, lds); break;                         \
        }                                                                                        \
    }
#define ZN_GEMMQ_LAYOUTS(S, KS, NSMAX, MINB)                                                     \
    ZN_GEMMQ_KERNEL(zn_sgemmq4##S##_nn_v, true, false, 16, KS, NSMAX, MINB)                      \
    ZN_GEMMQ_KERNEL(zn_sgemmq4##S##_nt_v, true, true, 16, KS, NSMAX, MINB)                       \
    ZN_GEMMQ_KERNEL(zn_sgemmq4##S##_tn_v, false, false, 16, KS, NSMAX, MINB)                     \
    ZN_GEMMQ_KERNEL(zn_sgemmq4##S##_nn, true, false, 4, KS, NSMAX, MINB)                         \
    ZN_GEMMQ_KERNEL(zn_sgemmq4##S##_nt, true, true, 4, KS, NSMAX, MINB)                          \
    ZN_GEMMQ_KERNEL(zn_sgemmq4##S##_tn, false, false, 4, KS, NSMAX, MINB)
ZN_GEMMQ_LAYOUTS(, 4, 8, 1)
ZN_GEMMQ_LAYOUTS(m, 4, 2, 4)
#define ZN_GEMMQ8_LAYOUTS                                                                        \
    ZN_GEMMQ_KERNEL(zn_sgemmq8_nn_v, true, false, 16, 8, 1, 1)                                   \
    ZN_GEMMQ_KERNEL(zn_sgemmq8_nt_v, true, true, 16, 8, 1, 1)                                    \
    ZN_GEMMQ_KERNEL(zn_sgemmq8_tn_v, false, false, 16, 8, 1, 1)                                  \
    ZN_GEMMQ_KERNEL(zn_sgemmq8_nn, true, false, 4, 8, 1, 1)                                      \
    ZN_GEMMQ_KERNEL(zn_sgemmq8_nt, true, true, 4, 8, 1, 1)                                       \
    ZN_GEMMQ_KERNEL(zn_sgemmq8_tn, false, false, 4, 8, 1, 1)
ZN_GEMMQ8_LAYOUTS

// Persistent plain GEMMs (gemm_persistent), 16-byte staging only:
// zn_sgemmp_<layout>_<tile>_v, for problems of several rounds of tiles.
#define ZN_GEMMP_KERNEL(NAME, BM, BN, BK, WM, WN, AK, BKC, MINB)                                 \
    extern "C" __global__ __launch_bounds__(WM *WN * 64, MINB) void NAME(ZnGemmArgs p) {        \
        __shared__ __attribute__((aligned(1024))) float lds[2 * (BM + BN) * BK];                 \
        switch (p.act) {                                                                         \
        case 1: gemm_persistent<BM, BN, BK, WM, WN, AK, BKC, 16, 16, 1>(p, lds); break;          \
        case 2: gemm_persistent<BM, BN, BK, WM, WN, AK, BKC, 16, 16, 2>(p, lds); break;          \
        case 3: gemm_persistent<BM, BN, BK, WM, WN, AK, BKC, 16, 16, 3>(p, lds); break;          \
        default: gemm_persistent<BM, BN, BK, WM, WN, AK, BKC, 16, 16, 0>(p, lds); break;         \
        }                                                                                        \
    }
#define ZN_GEMMP_TILE(TILE, BM, BN, BK, WM, WN, MINB)                                           \
    ZN_GEMMP_KERNEL(zn_sgemmp_nn_##TILE##_v, BM, BN, BK, WM, WN, true, false, MINB)             \
    ZN_GEMMP_KERNEL(zn_sgemmp_nt_##TILE##_v, BM, BN, BK, WM, WN, true, true, MINB)              \
    ZN_GEMMP_KERNEL(zn_sgemmp_tn_##TILE##_v, BM, BN, BK, WM, WN, false, false, MINB)

ZN_GEMMP_TILE(x, 256, 128, 16, 4, 2, 1)
ZN_GEMMP_TILE(l, 128, 128, 16, 2, 2, 3)  // 3 waves per SIMD: the TN form needs 145 VGPRs (at 4, it spilled)
ZN_GEMMP_TILE(n, 128, 64, 16, 2, 1, 1)
ZN_GEMMP_TILE(m, 64, 64, 32, 2, 2, 1)

// Persistent plain GEMMs with deferred stores (gemm_persistent_defer) on
// the 128x128 tile, 4 waves of 32x128: zn_sgemmpd_<layout>_l_v.  Each lane
// then holds 4 consecutive columns of C and stores them as one float4 (C5
// QK^T 178 -> 169 us against 4 waves of 64x64 storing float2s, 4-byte
// stores before the X-permuted B fragments).  (On 256x128 tiles of 64x64
// waves they ran at the same speed.)
#define ZN_GEMMPD_KERNEL(NAME, BM, BN, WM, WN, AK, BKC, KT)                                      \
    extern "C" __global__ __launch_bounds__(WM *WN * 64, 2) void NAME(ZnGemmArgs p) {           \
        __shared__ __attribute__((aligned(1024))) float lds[2 * (BM + BN) * 16];                 \
        gemm_persistent_defer<BM, BN, 16, WM, WN, AK, BKC, KT>(p, lds);                          \
    }
#define ZN_GEMMPD_TILE(TILE, BM, BN, WM, WN, KT, S)                                              \
    ZN_GEMMPD_KERNEL(zn_sgemmpd##S##_nn_##TILE##_v, BM, BN, WM, WN, true, false, KT)             \
    ZN_GEMMPD_KERNEL(zn_sgemmpd##S##_nt_##TILE##_v, BM, BN, WM, WN, true, true, KT)              \
    ZN_GEMMPD_KERNEL(zn_sgemmpd##S##_tn_##TILE##_v, BM, BN, WM, WN, false, false, KT)
ZN_GEMMPD_TILE(l, 128, 128, 4, 1, 0, )
// zn_sgemmpd4_<layout>_l_v: K of exactly 4 slices (C5 QK^T, K = 64)
ZN_GEMMPD_TILE(l, 128, 128, 4, 1, 4, 4)

// Split-K finish: C = act((accumulate ? C : 0) + sum over slices s = 0..S-1
// of ws[s] + bias[col or row]).  Slices are summed in ascending order, so results do not
// depend on scheduling.  Grid-stride over batch * m * n (float4 along n when
// n, ldc and C allow it).
__device__ __forceinline__ void splitk_reduce_body(const ZnReduceArgs &p, int64_t block, int64_t blocks) {
    const int64_t mn = (int64_t)p.m * p.n;
    const int vw = p.vec ? 4 : 1;
    const int64_t per_problem = mn / vw;
    const int64_t total = per_problem * p.batch;
    for (int64_t t = block * 256 + threadIdx.x; t < total; t += blocks * 256) {
        const int64_t b = t / per_problem;
        const int64_t e = (t - b * per_problem) * vw;  // element index within the problem
        const int64_t row = e / p.n, col = e - row * p.n;
        const float *src = p.ws + b * p.splits * mn + e;
        float *dst = p.c + b * p.stride_c + row * p.ldc + col;
        if (p.vec) {
            // up to 8 slices' loads in flight at once, added in slice order
            zn_f32x4 s = *reinterpret_cast<const zn_f32x4 *>(src);
            for (int z0 = 1; z0 < p.splits; z0 += 8) {
                zn_f32x4 x[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (z0 + u < p.splits) x[u] = *reinterpret_cast<const zn_f32x4 *>(src + (z0 + u) * mn);
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (z0 + u < p.splits) s = s + x[u];
            }
            zn_f32x4 v = s;
            if (p.accumulate) v = *reinterpret_cast<const zn_f32x4 *>(dst) + v;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float x = v[q];
                if (p.bias) x = x + p.bias[p.bias_rows ? row : col + q];
                v[q] = zn_activate(x, p.act);
            }
            *reinterpret_cast<zn_f32x4 *>(dst) = v;
        } else {
            float s = src[0];
            for (int z0 = 1; z0 < p.splits; z0 += 8) {
                float x[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (z0 + u < p.splits) x[u] = src[(z0 + u) * mn];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (z0 + u < p.splits) s = s + x[u];
            }
            float x = p.accumulate ? dst[0] + s : s;
            if (p.bias) x = x + p.bias[p.bias_rows ? row : col];
            dst[0] = zn_activate(x, p.act);
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void zn_splitk_reduce(ZnReduceArgs p) {
    splitk_reduce_body(p, blockIdx.x, gridDim.x);
}

// The bias gradient of a Dense backward as column sums (ZnColSumArgs), for
// the grouped launches that run without a prologue: workgroup `block` takes
// 16 columns; thread t sums the rows of splits t / 16, t / 16 + 16, ... of
// column t % 16 in row order (and copies them when asked), then 16 threads
// add each column's split sums in split order onto dst.  `lds` holds
// splits x 16 floats.
__device__ __forceinline__ void dense_colsum_body(const ZnColSumArgs &p, int block, float *lds) {
    const int t = threadIdx.x;
    const int col = block * 16 + (t & 15);
    for (int s = t >> 4; s < p.splits; s += 16) {
        float sum = 0.0f;
        if (col < p.n) {
            const int r1 = min(p.rows, (s + 1) * p.per);
            for (int r = s * p.per; r < r1; ++r) {
                const float v = p.src[(int64_t)r * p.n + col];
                if (p.copy) p.copy[(int64_t)r * p.n + col] = v;
                sum = sum + v;
            }
        }
        lds[s * 16 + (t & 15)] = sum;
    }
    __syncthreads();
    if (t < 16 && col < p.n) {
        float total = lds[t];
        for (int s = 1; s < p.splits; ++s) total = total + lds[s * 16 + t];
        p.dst[col] = p.dst[col] + total;
    }
}

// Dense backward GEMMs in one launch (ZnDenseBwdArgs): grad_input = gaa . W^T
// (NT), grad_weights = input^T . gaa (TN), and the bias gradient (the reduce
// of the prologue's partials, or the column sums themselves).  _v: both
// GEMMs stage with 16-byte loads.
#define ZN_DENSE_BWD_KERNEL(SUFFIX, W)                                                              \
    extern "C" __global__ __launch_bounds__(256, 1) void zn_dense_bwd_m##SUFFIX(ZnDenseBwdArgs p) { \
        __shared__ float colsum_lds[kMaxColSumSplits * 16];                                          \
        const int b = blockIdx.x;                                                                    \
        if (b < p.wg_nt)                                                                             \
            gemm_tile_dma<64, 64, 32, 2, 2, true, true, W, W>(p.nt, b);                             \
        else if (b < p.wg_nt + p.wg_tn)                                                              \
            gemm_tile_dma<64, 64, 32, 2, 2, false, false, W, W>(p.tn, b - p.wg_nt);                 \
        else if (p.wg_colsum)                                                                        \
            dense_colsum_body(p.colsum, b - p.wg_nt - p.wg_tn, colsum_lds);                          \
        else                                                                                         \
            splitk_reduce_body(p.bias, b - p.wg_nt - p.wg_tn, p.wg_bias);                           \
    }
ZN_DENSE_BWD_KERNEL(_v, 16)
ZN_DENSE_BWD_KERNEL(, 4)

// The same grouping on 32x32 tiles whose four waves split K (gemm_ksplit):
// more, shorter workgroups for the small layers of an MLP.
#define ZN_DENSE_BWDK_KERNEL(SUFFIX, W)                                                             \
    extern "C" __global__ __launch_bounds__(256, 1) void zn_dense_bwd_k##SUFFIX(ZnDenseBwdArgs p) { \
        __shared__ __attribute__((aligned(1024))) float lds[4 * 2 * (32 + 32) * 32];                 \
        const int b = blockIdx.x;                                                                    \
        if (b < p.wg_nt)                                                                             \
            gemm_ksplit<32, 32, 32, 4, true, true, W, W, 0>(p.nt, lds, b);                           \
        else if (b < p.wg_nt + p.wg_tn)                                                              \
            gemm_ksplit<32, 32, 32, 4, false, false, W, W, 0>(p.tn, lds, b - p.wg_nt);               \
        else if (p.wg_colsum)                                                                        \
            dense_colsum_body(p.colsum, b - p.wg_nt - p.wg_tn, lds);                                 \
        else                                                                                         \
            splitk_reduce_body(p.bias, b - p.wg_nt - p.wg_tn, p.wg_bias);                           \
    }
ZN_DENSE_BWDK_KERNEL(_v, 16)
ZN_DENSE_BWDK_KERNEL(, 4)
