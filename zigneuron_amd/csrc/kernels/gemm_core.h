// fp32 GEMM core for gfx950 (CDNA4) on the fp32 matrix cores: the device
// code shared by the GEMM (gemm_f32.hip) and convolution (conv_f32.hip)
// code objects.
//
// One MFMA core serves the three layouts of ZigNeuron's Backend.matMul family
// (NN: src/backend.zig:169, TN: :298, NT: :310), the fused bias+activation
// epilogues (:200-295) and a strided-batched grid (blockIdx.y = problem).
//
// Structure of one workgroup (BM x BN macro tile, WM x WN waves):
//  * Two LDS stages, one barrier per BK slice: slice kt + 1 is loaded while
//    slice kt is multiplied.  Operands go straight from HBM into LDS with
//    buffer_load ... lds (no staging registers, no LDS stores): 16-byte
//    loads for aligned operands (the _v kernels), 4-byte loads otherwise.
//  * Each operand keeps its global layout in LDS: a K-contiguous operand (A
//    of NN/NT, B of NT) is stored by rows of x, an X-contiguous one (A of TN,
//    B of NN/TN) by rows of k.  NN, NT and TN differ only in how lanes read
//    fragments, so no transposing LDS writes are needed.
//  * v_mfma_f32_32x32x2f32: a 32x32 fp32 block per instruction, K = 2 split
//    over the two lane halves.  The K order inside a group of 8 is permuted
//    so that lane half h, step t covers k = 8g + 4h + t; a K-contiguous
//    fragment is then one 16-byte LDS read per block.
//  * For an X-contiguous operand the 32 lanes of a block own FX consecutive
//    tile rows/cols (row = FX*i + f), so their fragment is one FX-wide LDS
//    read and, for B, their output columns are FX-wide vector stores.
//  * Edges (ragged M, N, K) are zero-filled in LDS: masked lanes carry an
//    out-of-range buffer offset and read (or DMA) zeros, so the load path has
//    no branches; zero products leave the sums unchanged, and stores are
//    predicated.
//  * Split-K: blockIdx.z selects a K range; partial sums go to a workspace
//    and zn_splitk_reduce adds them in slice order (deterministic).

#ifndef ZN_GEMM_CORE_H
#define ZN_GEMM_CORE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../zn_kernel_args.h"

#include "zn_mfma_stage.h"
#include "zn_activation.h"

namespace {

// Where the B operand of a GEMM comes from (gemm_tile_dma's G):
enum ZnGather {
    kGNone = 0,        // a plain matrix
    kGIm2col = 1,      // implicit im2col of an NCHW batch, element gather (ConvGatherStage)
    kGIm2col4 = 2,     // the same, 4-pixel 16-byte gather (ConvGather16Stage)
    kGTransposed = 3,  // transposed convolution of grad_output rows (ConvTGatherStage)
    kGWeight = 4,      // col of a weight gradient (ConvWGatherStage)
    kGNhwc = 5,        // implicit im2col of an NHWC batch, 4-channel 16-byte gather (ConvNhwcGatherStage)
    kGNhwcW = 6,       // col of a weight gradient from an NHWC batch, X-contiguous (ConvNhwcWGatherStage)
};

__device__ __forceinline__ float zn_activate(float v, int act) {
    switch (act) {
    case 1: return v > 0.0f ? v : 0.0f;               // relu   (src/backend.zig:239-240)
    case 2: return 1.0f / (1.0f + expf(-v));          // sigmoid (src/backend.zig:264-265)
    case 3: return tanhf(v);                          // tanh   (src/backend.zig:289-290)
    default: return v;
    }
}

// x / d for 0 <= x < 2^31 with (mul, shift) as stored in ZnConvGeom
// (Granlund & Montgomery 1994, Theorem 4.2, with 31-bit dividends).
__device__ __forceinline__ int zn_udiv(int x, uint32_t mul, uint32_t shift) {
    return (int)(((uint64_t)(uint32_t)x * mul) >> (31 + shift));
}

// Implicit-GEMM convolution operand: the X-contiguous tile [BK][BN] of the
// virtual im2col matrix, element (k, n) gathered with 4-byte loads from the
// NCHW input (out-of-image taps and out-of-problem elements read zero).
//
// When BN is a whole number of waves wide and every wave keeps the same BN
// columns for all of its loads (kFixedN), a lane's output pixel n is fixed
// for the whole tile: its (oh, ow) decode is done once (Lane), and the filter
// tap of each load is uniform across the wave, decoded on the scalar unit.
// Otherwise (BN = 32) every element is decoded per lane.
template <int BN, int BK, int NT>
struct ConvGatherStage {
    static constexpr int kFloats = BN * BK;
    static constexpr int kInsts = kFloats / kWave;
    static constexpr int kWaves = NT / kWave;
    static constexpr int kPerWave = kInsts / kWaves;
    static_assert(kInsts % kWaves == 0 && kPerWave >= 1, "load blocks must split evenly over waves");
    static constexpr int kRowWaves = BN / kWave;  // wave loads per k row
    static constexpr bool kFixedN = BN % kWave == 0 && kWaves % kRowWaves == 0;

    struct Lane {
        int ih0, iw0;  // top-left input tap of this lane's output pixel
        int base;      // ih0 * in_w + iw0
        bool ok;       // the pixel lies inside the problem
    };

    __device__ static __forceinline__ Lane lane_setup(const ZnConvGeom &g, int n0, int nmax, int wave, int lane) {
        Lane l;
        const int n = n0 + (kFixedN ? (wave % kRowWaves) * kWave : 0) + lane;
        const int oh = n / g.out_w, ow = n - oh * g.out_w;
        l.ih0 = oh * g.stride_h - g.pad_h;
        l.iw0 = ow * g.stride_w - g.pad_w;
        l.base = l.ih0 * g.in_w + l.iw0;
        l.ok = n < nmax;
        return l;
    }

    __device__ static __forceinline__ void load(__amdgpu_buffer_rsrc_t rsrc, float *lds, int p0, uint32_t off) {
        const uint32_t lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(zn_lds_void *)(lds + p0));
        asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                     :
                     : "s"(lds_addr), "v"(off), "s"(rsrc)
                     : "memory");
    }

    // Filter tap of im2col column k: input channel, kernel row and column.
    __device__ static __forceinline__ void decode_k(const ZnConvGeom &g, int k, int &ic, int &kh, int &kw) {
        const int q = zn_udiv(k, g.div1_mul, g.div1_shift);
        const int r = k - q * g.div1;
        const int kpos = g.k_order == 0 ? q : r;
        ic = g.k_order == 0 ? r : q;
        kh = zn_udiv(kpos, g.kw_mul, g.kw_shift);
        kw = kpos - kh * g.k_w;
    }

    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, float *lds, const ZnConvGeom &g,
                                                 const Lane &ln, int n0, int k0, int nmax, int kmax, int wave,
                                                 int lane) {
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int row = j * kWaves + wave;  // wave-uniform
            const int p0 = row * kWave;
            uint32_t off;
            if constexpr (kFixedN) {
                const int k = k0 + row / kRowWaves;  // wave-uniform
                int ic, kh, kw;
                decode_k(g, k, ic, kh, kw);
                const int ih = ln.ih0 + kh, iw = ln.iw0 + kw;
                const bool ok = ln.ok && k < kmax && (unsigned)ih < (unsigned)g.in_h && (unsigned)iw < (unsigned)g.in_w;
                off = ok ? (uint32_t)(ln.base + (ic * g.in_h + kh) * g.in_w + kw) * 4u : kOutOfRange;
            } else {
                const int pos = p0 + lane;
                const int k = k0 + pos / BN;
                const int n = n0 + pos % BN;
                int ic, kh, kw;
                decode_k(g, k, ic, kh, kw);
                const int oh = zn_udiv(n, g.ow_mul, g.ow_shift), ow = n - oh * g.out_w;
                const int ih = oh * g.stride_h - g.pad_h + kh;
                const int iw = ow * g.stride_w - g.pad_w + kw;
                const bool ok = n < nmax && k < kmax && (unsigned)ih < (unsigned)g.in_h && (unsigned)iw < (unsigned)g.in_w;
                off = ok ? (uint32_t)((ic * g.in_h + ih) * g.in_w + iw) * 4u : kOutOfRange;
            }
            load(rsrc, lds, p0, off);
        }
    }
};

// Tile coordinates and split-K slice of this workgroup: optional XCD-
// contiguous remap, then groups of `group_m` tile rows (group_m = 1 is plain
// row-major order).  Workgroups go to the 8 XCDs round-robin by linear id,
// and each XCD has its own L2.  xcd_remap 2 (split-K, one problem): the
// (slice, tile) pairs are numbered slice-major and each XCD takes a
// contiguous run of them, so the tiles of one K slice, which read the same
// rows of A and B, share one L2 instead of fetching them once per XCD.
// `wg` >= 0 (a grouped launch) is this workgroup's index within its problem,
// which is unsplit.
__device__ __forceinline__ void tile_coords(const ZnGemmArgs &p, int &tm, int &tn, int &slice, int wg = -1) {
    int pid = wg >= 0 ? wg : (int)blockIdx.x;
    slice = wg >= 0 ? 0 : (int)blockIdx.z;
    const int ntiles = p.tiles_m * p.tiles_n;
    if (p.xcd_remap == 1) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
    if (p.xcd_remap == 2) {
        const int lin = blockIdx.x + ntiles * blockIdx.z;  // gridDim.y == 1
        const int total = ntiles * p.splits, per = total >> 3, extra = total & 7;
        const int xcd = lin & 7;
        const int seq = xcd * per + min(xcd, extra) + (lin >> 3);
        slice = seq / ntiles;
        pid = seq - slice * ntiles;
    }
    const int group_span = p.group_m * p.tiles_n;
    const int first_m = (pid / group_span) * p.group_m;
    const int gsize = min(p.tiles_m - first_m, p.group_m);
    const int in_group = pid % group_span;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// The convolution operand with 16-byte loads, for stride_w == 1 and
// out_w % 4 == 0: lane L of a wave instruction stages a chunk of 4
// neighbouring output pixels (one output row, so 4 consecutive input
// columns) of one filter tap.  A lane's pixel chunk is fixed for the whole
// tile (Lane); its tap changes with the instruction and is decoded per lane.
// Chunks wholly inside the image are one DMA.  A chunk that straddles the
// left or right padding is DMAed as zeros (out-of-range offset), and the lane
// loads its in-image elements with ordinary guarded loads and writes the
// chunk into LDS after its own DMA has landed (patch, before the barrier), so
// no access ever leaves the image.
template <int BN, int BK, int NT>
struct ConvGather16Stage {
    static constexpr int kFloats = BN * BK;
    static constexpr int kPerInst = 4 * kWave;  // 256 floats per wave instruction
    static constexpr int kInsts = kFloats / kPerInst;
    static constexpr int kWaves = NT / kWave;
    static constexpr int kPerWave = kInsts / kWaves;
    static_assert(kInsts % kWaves == 0 && kPerWave >= 1, "load blocks must split evenly over waves");
    static_assert(kPerInst % BN == 0, "a wave instruction covers whole k rows");
    static constexpr int kRowsPerInst = kPerInst / BN;

    struct Lane {
        int ih0, iw0;  // top-left input tap of the chunk's first pixel
        int kl;        // k row of this lane within a wave instruction
        bool ok;       // the chunk lies inside the problem
    };
    struct Patch {
        zn_f32x4 v[kPerWave];
        uint32_t mask;  // bit j: instruction j's chunk needs the patch
    };

    __device__ static __forceinline__ Lane lane_setup(const ZnConvGeom &g, int n0, int nmax, int lane) {
        Lane l;
        const int n = n0 + (4 * lane) % BN;  // first pixel of the chunk (n0 and out_w are multiples of 4)
        const int oh = n / g.out_w, ow = n - oh * g.out_w;
        l.ih0 = oh * g.stride_h - g.pad_h;
        l.iw0 = ow - g.pad_w;  // stride_w == 1
        l.kl = (4 * lane) / BN;
        l.ok = n < nmax;
        return l;
    }

    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, const float *image, float *lds,
                                                 const ZnConvGeom &g, const Lane &ln, int k0, int kmax, int wave,
                                                 int lane, Patch &pt) {
        pt.mask = 0;
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int row = j * kWaves + wave;  // wave-uniform
            const int p0 = row * kPerInst;
            const int k = k0 + row * kRowsPerInst + ln.kl;
            int ic, kh, kw;
            ConvGatherStage<BN, BK, NT>::decode_k(g, k, ic, kh, kw);
            const int ih = ln.ih0 + kh, iws = ln.iw0 + kw;
            const bool row_ok = ln.ok && k < kmax && (unsigned)ih < (unsigned)g.in_h;
            const bool full = row_ok && iws >= 0 && iws + 3 < g.in_w;
            const int row_off = (ic * g.in_h + ih) * g.in_w;
            const uint32_t off = full ? (uint32_t)(row_off + iws) * 4u : kOutOfRange;
            const uint32_t lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(zn_lds_void *)(lds + p0));
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                         :
                         : "s"(lds_addr), "v"(off), "s"(rsrc)
                         : "memory");
            pt.v[j] = zn_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if (row_ok && !full && iws + 3 >= 0 && iws < g.in_w) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if ((unsigned)(iws + e) < (unsigned)g.in_w) pt.v[j][e] = image[row_off + iws + e];
                pt.mask |= 1u << j;
            }
        }
    }

    // After this wave's DMA has landed: write the patched chunks.
    __device__ static __forceinline__ void apply(float *lds, const Patch &pt, int wave, int lane) {
        if (!pt.mask) return;
#pragma unroll
        for (int j = 0; j < kPerWave; ++j)
            if (pt.mask & (1u << j))
                *reinterpret_cast<zn_f32x4 *>(lds + (j * kWaves + wave) * kPerInst + 4 * lane) = pt.v[j];
    }
};

// The transposed-convolution operand (the input gradient of a stride-1
// convolution as an implicit GEMM): B[n][k] with n = input pixel (ih, iw)
// and k = (kh*k_w + kw)*OC + oc is grad_output[(ih + pad_h - kh, iw + pad_w -
// kw)][oc], grad_output read as [OH*OW][OC] rows (the reading of
// cpuConv2dBackwardIm2col).  The operand is K-contiguous (stored [BN][BK],
// swizzled like DmaStage), and a 16-byte chunk is 4 consecutive oc of one
// grad_output row (OC % 4 == 0), so each chunk is either wholly inside the
// output image or wholly outside (zeros): no patching.  ZnConvGeom fields as
// used here: channels = OC, in_h x in_w = OH x OW (the gathered image),
// out_w = W (decodes n), div1 = OC, k_w, pad as in the forward.
template <int BN, int BK, int NT>
struct ConvTGatherStage {
    typedef DmaStage<BN, BK, NT, true, 16> Layout;
    static constexpr int kPerWave = Layout::kPerWave;
    static constexpr int kWaves = NT / kWave;

    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, float *lds, const ZnConvGeom &g,
                                                 int n0, int k0, int nmax, int kmax, int wave, int lane) {
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int p0 = (j * kWaves + wave) * Layout::kPerInst;
            const int pos = p0 + 4 * lane;
            const int row = pos / BK;
            const int c = ((pos % BK) / 4) ^ Layout::swz(row);
            const int n = n0 + row, k = k0 + 4 * c;
            const int ih = zn_udiv(n, g.ow_mul, g.ow_shift), iw = n - ih * g.out_w;
            const int khw = zn_udiv(k, g.div1_mul, g.div1_shift);
            const int oc = k - khw * g.div1;
            const int kh = zn_udiv(khw, g.kw_mul, g.kw_shift), kw = khw - kh * g.k_w;
            const int oh = ih + g.pad_h - kh, ow = iw + g.pad_w - kw;
            const bool ok = n < nmax && k < kmax && (unsigned)oh < (unsigned)g.in_h && (unsigned)ow < (unsigned)g.in_w;
            const uint32_t off = ok ? (uint32_t)((oh * g.in_w + ow) * g.channels + oc) * 4u : kOutOfRange;
            const uint32_t lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(zn_lds_void *)(lds + p0));
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                         :
                         : "s"(lds_addr), "v"(off), "s"(rsrc)
                         : "memory");
        }
    }
};

// The weight-gradient operand of a convolution with stride_w == 1 and
// out_w % 4 == 0, without the col buffer: B[k][n] = col[k][n], k = output
// pixel over `images` images (b*OH*OW + oh*OW + ow), n = im2col tap
// (kh*k_w + kw)*C + ic, i.e. input[b][ic][oh*stride_h - pad_h + kh][ow -
// pad_w + kw].  The operand is K-contiguous (stored [BN][BK], swizzled like
// DmaStage): a 16-byte chunk is 4 consecutive k, i.e. 4 neighbouring output
// pixels of one output row, which read 4 consecutive input columns of one
// tap.  A lane's tap and chunk column are fixed for the whole tile (Lane);
// its pixels move with k0.  Chunks that straddle the left or right padding
// are DMAed as zeros and patched like ConvGather16Stage's.
template <int BN, int BK, int NT>
struct ConvWGatherStage {
    typedef DmaStage<BN, BK, NT, true, 16> Layout;
    static constexpr int kNoRow = -(1 << 30);  // plus any oh*stride_h stays negative
    static constexpr int kPerWave = Layout::kPerWave;
    static constexpr int kWaves = NT / kWave;

    struct Lane {
        int tap_off[kPerWave];  // ic*H*W + (kh - pad_h)*W + (kw - pad_w), relative to the pixel's (oh*sh, ow)
        int dh[kPerWave];       // kh - pad_h; kNoRow for a tap past the problem (never in the image)
        int dw[kPerWave];       // kw - pad_w
        int kc[kPerWave];       // first k of the chunk, relative to k0
    };
    struct Patch {
        zn_f32x4 v[kPerWave];
        uint32_t mask;
    };

    __device__ static __forceinline__ Lane lane_setup(const ZnConvGeom &g, int n0, int nmax, int wave, int lane) {
        Lane l;
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int pos = (j * kWaves + wave) * Layout::kPerInst + 4 * lane;
            const int row = pos / BK;
            const int n = n0 + row;
            int ic, kh, kw;
            ConvGatherStage<BN, BK, NT>::decode_k(g, n, ic, kh, kw);
            l.dh[j] = n < nmax ? kh - g.pad_h : kNoRow;
            l.dw[j] = kw - g.pad_w;
            l.tap_off[j] = (ic * g.in_h + kh - g.pad_h) * g.in_w + kw - g.pad_w;
            l.kc[j] = 4 * (((pos % BK) / 4) ^ Layout::swz(row));
        }
        return l;
    }

    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, const float *image, float *lds,
                                                 const ZnConvGeom &g, const Lane &ln, int k0, int kmax, int wave,
                                                 int lane, Patch &pt) {
        pt.mask = 0;
        const int plane = g.channels * g.in_h * g.in_w;
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int p0 = (j * kWaves + wave) * Layout::kPerInst;
            const int k = k0 + ln.kc[j];
            const int q = zn_udiv(k, g.ow_mul, g.ow_shift), ow = k - q * g.out_w;
            const int b = zn_udiv(q, g.oh_mul, g.oh_shift), oh = q - b * g.out_h;
            const int ohs = oh * g.stride_h;
            const int ih = ohs + ln.dh[j], iws = ow + ln.dw[j];
            const bool row_ok = k < kmax && (unsigned)ih < (unsigned)g.in_h;
            const bool full = row_ok && iws >= 0 && iws + 3 < g.in_w;
            const int src = b * plane + ln.tap_off[j] + ohs * g.in_w + ow;  // = b*plane + (ic*H + ih)*W + iws
            const uint32_t off = full ? (uint32_t)src * 4u : kOutOfRange;
            const uint32_t lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(zn_lds_void *)(lds + p0));
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                         :
                         : "s"(lds_addr), "v"(off), "s"(rsrc)
                         : "memory");
            pt.v[j] = zn_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if (row_ok && !full && iws + 3 >= 0 && iws < g.in_w) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if ((unsigned)(iws + e) < (unsigned)g.in_w) pt.v[j][e] = image[src + e];
                pt.mask |= 1u << j;
            }
        }
    }

    // After this wave's DMA has landed: write the patched chunks.
    __device__ static __forceinline__ void apply(float *lds, const Patch &pt, int wave, int lane) {
        if (!pt.mask) return;
#pragma unroll
        for (int j = 0; j < kPerWave; ++j)
            if (pt.mask & (1u << j))
                *reinterpret_cast<zn_f32x4 *>(lds + (j * kWaves + wave) * Layout::kPerInst + 4 * lane) = pt.v[j];
    }
};

// The implicit im2col operand of an NHWC image batch: B[n][k] with n = output
// pixel (oh, ow) and k = (kh*k_w + kw)*C + ic (the im2col K order) is
// image[(oh*stride_h - pad_h + kh, ow*stride_w - pad_w + kw)][ic].  The
// operand is K-contiguous (stored [BN][BK], swizzled like DmaStage): a 16-byte
// chunk is 4 consecutive channels of one pixel (C % 4 == 0), so it is either
// wholly inside the image or wholly padding (zeros), at any stride.
// ZnConvGeom as in the forward: channels = C, in_h x in_w, out_w decodes n,
// div1 = C, k_w.
template <int BN, int BK, int NT>
struct ConvNhwcGatherStage {
    typedef DmaStage<BN, BK, NT, true, 16> Layout;
    static constexpr int kPerWave = Layout::kPerWave;
    static constexpr int kWaves = NT / kWave;

    // A lane's output pixel and chunk column are fixed for the whole tile:
    // decoded once.  ih0/iw0: the pixel's top-left input tap (ih0 = kNoRow
    // for a pixel past the problem, so no tap is ever inside the image).
    struct Lane {
        int ih0[kPerWave], iw0[kPerWave];
        int kc[kPerWave];  // first k of the chunk, relative to k0
    };
    static constexpr int kNoRow = -(1 << 30);

    __device__ static __forceinline__ Lane lane_setup(const ZnConvGeom &g, int n0, int nmax, int wave, int lane) {
        Lane l;
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int pos = (j * kWaves + wave) * Layout::kPerInst + 4 * lane;
            const int row = pos / BK;
            const int n = n0 + row;
            const int oh = zn_udiv(n, g.ow_mul, g.ow_shift), ow = n - oh * g.out_w;
            l.ih0[j] = n < nmax ? oh * g.stride_h - g.pad_h : kNoRow;
            l.iw0[j] = ow * g.stride_w - g.pad_w;
            l.kc[j] = 4 * (((pos % BK) / 4) ^ Layout::swz(row));
        }
        return l;
    }

    // tap_uniform (C % BK == 0): the slice [k0, k0 + BK) lies in one filter
    // tap, decoded once per slice on the scalar unit.
    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, float *lds, const ZnConvGeom &g,
                                                 const Lane &ln, int k0, int kmax, int wave, int lane) {
        int kh_u = 0, kw_u = 0, ic_u = 0;
        if (g.tap_uniform) {
            const int khw = zn_udiv(k0, g.div1_mul, g.div1_shift);
            ic_u = k0 - khw * g.div1;
            kh_u = zn_udiv(khw, g.kw_mul, g.kw_shift);
            kw_u = khw - kh_u * g.k_w;
        }
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int p0 = (j * kWaves + wave) * Layout::kPerInst;
            const int k = k0 + ln.kc[j];
            int kh, kw, ic;
            if (g.tap_uniform) {
                kh = kh_u;
                kw = kw_u;
                ic = ic_u + ln.kc[j];
            } else {
                const int khw = zn_udiv(k, g.div1_mul, g.div1_shift);
                ic = k - khw * g.div1;
                kh = zn_udiv(khw, g.kw_mul, g.kw_shift);
                kw = khw - kh * g.k_w;
            }
            const int ih = ln.ih0[j] + kh, iw = ln.iw0[j] + kw;
            const bool ok = k < kmax && (unsigned)ih < (unsigned)g.in_h && (unsigned)iw < (unsigned)g.in_w;
            const uint32_t off = ok ? (uint32_t)((ih * g.in_w + iw) * g.channels + ic) * 4u : kOutOfRange;
            const uint32_t lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(zn_lds_void *)(lds + p0));
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                         :
                         : "s"(lds_addr), "v"(off), "s"(rsrc)
                         : "memory");
        }
    }
};

// The col operand of a weight gradient from an NHWC image batch: B[k][n] =
// col[k][n] with k = output pixel over `images` images (b*OH*OW + oh*OW +
// ow) and n = im2col tap (kh*k_w + kw)*C + ic, i.e. image_b[(oh*stride_h -
// pad_h + kh, ow*stride_w - pad_w + kw)][ic].  X-contiguous (stored
// [BK][BN] like DmaStage): a 16-byte chunk is 4 consecutive channels of one
// tap at one pixel (C % 4 == 0), wholly inside the image or wholly padding,
// at any stride.  A lane's tap is fixed for the tile; its pixel moves with k0.
template <int BN, int BK, int NT>
struct ConvNhwcWGatherStage {
    typedef DmaStage<BN, BK, NT, false, 16> Layout;
    static constexpr int kPerWave = Layout::kPerWave;
    static constexpr int kWaves = NT / kWave;
    static_assert(Layout::kPerInst % BN == 0, "a wave instruction covers whole k rows");
    static constexpr int kRowsPerInst = Layout::kPerInst / BN;
    static constexpr int kNoRow = -(1 << 30);

    struct Lane {
        int dh, dw;   // kh - pad_h (kNoRow past the problem), kw - pad_w
        int tap_off;  // (kh - pad_h) * W * C + (kw - pad_w) * C + ic
        int kl;       // k row of this lane within a wave instruction
    };

    __device__ static __forceinline__ Lane lane_setup(const ZnConvGeom &g, int n0, int nmax, int lane) {
        Lane l;
        const int n = n0 + (4 * lane) % BN;
        const int khw = zn_udiv(n, g.div1_mul, g.div1_shift);
        const int ic = n - khw * g.div1;
        const int kh = zn_udiv(khw, g.kw_mul, g.kw_shift), kw = khw - kh * g.k_w;
        l.dh = n < nmax ? kh - g.pad_h : kNoRow;
        l.dw = kw - g.pad_w;
        l.tap_off = ((kh - g.pad_h) * g.in_w + (kw - g.pad_w)) * g.channels + ic;
        l.kl = (4 * lane) / BN;
        return l;
    }

    // byte offset of this lane's chunk of load j (a wave-uniform k row pair)
    // of the slice at k0, or kOutOfRange (padding, or k at or past kmax)
    __device__ static __forceinline__ uint32_t offset(const ZnConvGeom &g, const Lane &ln, int k0, int kmax, int wave,
                                                      int j) {
        const int plane = g.channels * g.in_h * g.in_w;
        const int row = j * kWaves + wave;  // wave-uniform
        const int k = k0 + row * kRowsPerInst + ln.kl;
        const int q = zn_udiv(k, g.ow_mul, g.ow_shift), ow = k - q * g.out_w;
        const int b = zn_udiv(q, g.oh_mul, g.oh_shift), oh = q - b * g.out_h;
        const int ohs = oh * g.stride_h, ows = ow * g.stride_w;
        const int ih = ohs + ln.dh, iw = ows + ln.dw;
        const bool ok = k < kmax && (unsigned)ih < (unsigned)g.in_h && (unsigned)iw < (unsigned)g.in_w;
        const int src = b * plane + (ohs * g.in_w + ows) * g.channels + ln.tap_off;
        return ok ? (uint32_t)src * 4u : kOutOfRange;
    }

    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, float *lds, const ZnConvGeom &g,
                                                 const Lane &ln, int k0, int kmax, int wave) {
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int p0 = (j * kWaves + wave) * Layout::kPerInst;
            const uint32_t off = offset(g, ln, k0, kmax, wave, j);
            const uint32_t lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(zn_lds_void *)(lds + p0));
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                         :
                         : "s"(lds_addr), "v"(off), "s"(rsrc)
                         : "memory");
        }
    }
};

// Epilogue of one macro tile: v = acc (+ C) (+ bias) -> act -> store.
// 32x32 accumulator layout: register r of lane (j = lane % 32, h = lane / 32)
// holds block row 8*(r/4) + 4*h + r%4, block column j.  A split-K slice
// stores its raw partial sums to the workspace instead.
// ACT >= 0: the activation is a template argument, one copy of the element
// loop per activation, entered once.  That keeps the executed code of a
// launch short for the small tiles (the instruction cache is cold for most
// small launches: alternating two small GEMM kernels cost 1.6 us per launch
// more than repeating one).  ACT = -1 reads it at run time; the 128x128 and
// 256x128 tiles keep that form (the specialised copies made the 8192^3 main
// loop 0.9-1.3% slower in NN and NT).
// STREAM: C is written with non-temporal stores (the persistent kernels,
// whose short-K problems are bound by writing C).
template <int BM, int BN, int WM, int WN, bool AK, bool BKC, int ACT, bool STREAM = false>
__device__ __forceinline__ void store_tile_act(const ZnGemmArgs &p, const zn_f32x16 (&acc)[BM / WM / 32][BN / WN / 32],
                                               int64_t bz, int m0, int n0, int wm0, int wn0, int lane, int slice) {
    constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
    float *gc = p.c + bz * p.stride_c;
    const bool split = p.splits > 1;
    if (split) gc = p.ws + ((int64_t)bz * p.splits + slice) * (int64_t)p.m * p.n;
    const int64_t ldc = split ? (int64_t)p.n : p.ldc;
    const bool accumulate = !split && p.accumulate;
    const int act = ACT >= 0 ? ACT : (split ? 0 : p.act);
    const int j = lane & 31;
    const int h = lane >> 5;
    const bool has_bias = !split && p.bias != nullptr;
    const bool col_bias = has_bias && !p.bias_rows;
    const bool row_bias = has_bias && p.bias_rows;
    float bias_v[FN];
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
        const int col = n0 + wn0 + (BKC ? 32 * fn + j : FN * j + fn);
        bias_v[fn] = (col_bias && col < p.n) ? p.bias[col] : 0.0f;
    }
    const bool vec_c = split ? (p.n % 4 == 0) : (p.vec_c != 0);
    const bool vec_store = !BKC && FN > 1 && vec_c && (n0 + wn0 + FN * j + FN <= p.n);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int bi = 8 * (r >> 2) + 4 * h + (r & 3);
            const int row = m0 + wm0 + (AK ? 32 * fm + bi : FM * bi + fm);
            if (row >= p.m) continue;
            float *crow = gc + (int64_t)row * ldc;
            const float rb = row_bias ? p.bias[row] : 0.0f;
            if constexpr (!BKC && FN > 1) {
                if (vec_store) {
                    typedef typename FVec<FN>::type VT;
                    VT *dst = reinterpret_cast<VT *>(crow + n0 + wn0 + FN * j);
                    VT v;
                    if (accumulate) v = *dst;
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn) {
                        float x = acc[fm][fn][r];
                        if (accumulate) x = v[fn] + x;
                        if (has_bias) x = x + (row_bias ? rb : bias_v[fn]);
                        v[fn] = zn_activate(x, act);
                    }
                    if constexpr (STREAM)
                        __builtin_nontemporal_store(v, dst);
                    else
                        *dst = v;
                    continue;
                }
            }
            {
#pragma unroll
                for (int fn = 0; fn < FN; ++fn) {
                    const int col = n0 + wn0 + (BKC ? 32 * fn + j : FN * j + fn);
                    if (col >= p.n) continue;
                    float x = acc[fm][fn][r];
                    if (accumulate) x = crow[col] + x;
                    if (has_bias) x = x + (row_bias ? rb : bias_v[fn]);
                    if constexpr (STREAM)
                        __builtin_nontemporal_store(zn_activate(x, act), &crow[col]);
                    else
                        crow[col] = zn_activate(x, act);
                }
            }
        }
    }
}

// Epilogue of gemm_tile_pinned.  A tile with nothing to add or apply (a
// plain GEMM, or a split-K slice's raw partial sums) takes a short path of
// stores, predicated on the edges of C; everything else goes through
// store_tile_act with the activation as a template argument.  One-round
// problems run the epilogue once per CU, all at the end and with a cold
// instruction cache, so the length of the executed code shows:
// 2048x2048x1024 NN on 128x128 tiles took 72.4 us with this path, 77.3 us
// through store_tile_act<ACT = 0> and 87.5 us through the run-time
// activation form.
template <int BM, int BN, int WM, int WN, bool AK, bool BKC>
__device__ __forceinline__ void store_tile_fast(const ZnGemmArgs &p, const zn_f32x16 (&acc)[BM / WM / 32][BN / WN / 32],
                                                int64_t bz, int m0, int n0, int wm0, int wn0, int lane, int slice) {
    constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
    const bool split = p.splits > 1;
    if (split || (!p.accumulate && !p.bias && p.act == 0)) {
        float *gc = split ? p.ws + ((int64_t)bz * p.splits + slice) * (int64_t)p.m * p.n : p.c + bz * p.stride_c;
        const int64_t ldc = split ? (int64_t)p.n : p.ldc;
        const bool vec_c = split ? p.n % 4 == 0 : p.vec_c != 0;
        const bool full_n = n0 + BN <= p.n;
        const int j = lane & 31, h = lane >> 5;
        const int c0 = n0 + wn0 + (BKC ? j : FN * j);  // this lane's first column
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int bi = 8 * (r >> 2) + 4 * h + (r & 3);
                const int row = m0 + wm0 + (AK ? 32 * fm + bi : FM * bi + fm);
                if (row >= p.m) continue;
                float *crow = gc + (int64_t)row * ldc;
                if constexpr (BKC || FN == 1) {
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn)
                        if (full_n || c0 + 32 * fn < p.n) crow[c0 + 32 * fn] = acc[fm][fn][r];
                } else {
                    if (vec_c && (full_n || c0 + FN <= p.n)) {
                        typedef typename FVec<FN>::type VT;
                        VT v;
#pragma unroll
                        for (int fn = 0; fn < FN; ++fn) v[fn] = acc[fm][fn][r];
                        *reinterpret_cast<VT *>(crow + c0) = v;
                    } else {
#pragma unroll
                        for (int fn = 0; fn < FN; ++fn)
                            if (c0 + fn < p.n) crow[c0 + fn] = acc[fm][fn][r];
                    }
                }
            }
        return;
    }
    switch (split ? 0 : p.act) {
    case 1: store_tile_act<BM, BN, WM, WN, AK, BKC, 1>(p, acc, bz, m0, n0, wm0, wn0, lane, slice); break;
    case 2: store_tile_act<BM, BN, WM, WN, AK, BKC, 2>(p, acc, bz, m0, n0, wm0, wn0, lane, slice); break;
    case 3: store_tile_act<BM, BN, WM, WN, AK, BKC, 3>(p, acc, bz, m0, n0, wm0, wn0, lane, slice); break;
    default: store_tile_act<BM, BN, WM, WN, AK, BKC, 0>(p, acc, bz, m0, n0, wm0, wn0, lane, slice); break;
    }
}

template <int BM, int BN, int WM, int WN, bool AK, bool BKC>
__device__ __forceinline__ void store_tile(const ZnGemmArgs &p, const zn_f32x16 (&acc)[BM / WM / 32][BN / WN / 32],
                                           int64_t bz, int m0, int n0, int wm0, int wn0, int lane, int slice) {
    if constexpr (BM * BN >= 128 * 128) {
        store_tile_act<BM, BN, WM, WN, AK, BKC, -1>(p, acc, bz, m0, n0, wm0, wn0, lane, slice);
        return;
    }
    switch (p.splits > 1 ? 0 : p.act) {  // split-K slices store raw partial sums
    case 1: store_tile_act<BM, BN, WM, WN, AK, BKC, 1>(p, acc, bz, m0, n0, wm0, wn0, lane, slice); break;
    case 2: store_tile_act<BM, BN, WM, WN, AK, BKC, 2>(p, acc, bz, m0, n0, wm0, wn0, lane, slice); break;
    case 3: store_tile_act<BM, BN, WM, WN, AK, BKC, 3>(p, acc, bz, m0, n0, wm0, wn0, lane, slice); break;
    default: store_tile_act<BM, BN, WM, WN, AK, BKC, 0>(p, acc, bz, m0, n0, wm0, wn0, lane, slice); break;
    }
}

// The GEMM main loop: two LDS stages filled by DMA (WA/WB = 16: 16-byte
// loads for aligned operands, 4: 4-byte loads otherwise; G != kGNone gathers
// B, ZnGather).  Iteration kt waits
// for its stage (vmcnt(0) + barrier), refills the other stage with slice
// kt + 1, then computes slice kt while that load is in flight.
template <int BM, int BN, int BK, int WM, int WN, bool AK, bool BKC, int WA, int WB, int G = kGNone>
__device__ __forceinline__ void gemm_tile_dma(const ZnGemmArgs &p, int wg = -1) {
    constexpr bool CONV = G == kGIm2col || G == kGIm2col4;
    constexpr int GW = G == kGIm2col4 ? 16 : 4;
    constexpr bool CONVT = G == kGTransposed, CONVW = G == kGWeight, NHWC = G == kGNhwc, NHWCW = G == kGNhwcW;
    constexpr int NT = WM * WN * kWave;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
    static_assert(!CONV || (!BKC && WB == 4), "the convolution operand is X-contiguous and gathered");
    static_assert(!CONVT || (BKC && WB == 16), "the transposed-convolution operand is K-contiguous");
    static_assert(!CONVW || (BKC && WB == 16), "the weight-gradient operand is K-contiguous");
    static_assert(!NHWC || (BKC && WB == 16), "the NHWC im2col operand is K-contiguous");
    static_assert(!NHWCW || (!BKC && WB == 16), "the NHWC weight-gradient operand is X-contiguous");
    typedef DmaStage<BM, BK, NT, AK, WA> SA;
    typedef DmaStage<BN, BK, NT, BKC, WB> SB;
    typedef ConvGatherStage<BN, BK, NT> SC;
    typedef ConvGather16Stage<BN, BK, NT> SC16;
    typedef ConvTGatherStage<BN, BK, NT> ST;
    typedef ConvWGatherStage<BN, BK, NT> SW;
    typedef ConvNhwcGatherStage<BN, BK, NT> SN;
    typedef ConvNhwcWGatherStage<BN, BK, NT> SNW;
    __shared__ __attribute__((aligned(1024))) float lds_a[2][SA::kFloats];
    __shared__ __attribute__((aligned(1024))) float lds_b[2][SB::kFloats];

    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;
    int tm, tn, slice;
    tile_coords(p, tm, tn, slice, wg);
    const int m0 = tm * BM, n0 = tn * BN;
    const int64_t bz = blockIdx.y;  // 0 in grouped launches
    const float *ga = p.a + bz * p.stride_a;
    const float *gb = p.b + bz * p.stride_b;

    zn_f32x16 acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0.0f;

    const int kbeg = slice * p.k_chunk;
    const int kend = min(p.k, kbeg + p.k_chunk);
    const int ktiles = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int lda = (int)p.lda, ldb = (int)p.ldb;
    // 16-byte staging reads whole float4s: the last row's extent is rounded
    // up to 4 floats (rows that are whole float4s, or packed with a zero tail)
    constexpr int RA = WA == 16 ? 3 : 0, RB = WB == 16 ? 3 : 0;
    const uint32_t a_bytes = (uint32_t)(AK ? (p.m - 1) * lda + ((p.k + RA) & ~RA) : (p.k - 1) * lda + ((p.m + RA) & ~RA)) * 4u;
    const uint32_t b_bytes =
        (CONVW || NHWCW) ? (uint32_t)(p.conv.images * p.conv.channels * p.conv.in_h * p.conv.in_w) * 4u
        : (CONV || CONVT || NHWC) ? (uint32_t)(p.conv.channels * p.conv.in_h * p.conv.in_w) * 4u
             : (uint32_t)(BKC ? (p.n - 1) * ldb + ((p.k + RB) & ~RB) : (p.k - 1) * ldb + ((p.n + RB) & ~RB)) * 4u;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(ga, a_bytes);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(gb, b_bytes);

    typename SC::Lane cl{};
    typename SC16::Lane cl16{};
    typename SC16::Patch patch;
    patch.mask = 0;
    if constexpr (CONV && GW == 4 && SC::kFixedN) cl = SC::lane_setup(p.conv, n0, p.n, wave, lane);
    if constexpr (CONV && GW == 16) cl16 = SC16::lane_setup(p.conv, n0, p.n, lane);
    typename SW::Lane clw{};
    typename SW::Patch wpatch;
    wpatch.mask = 0;
    if constexpr (CONVW) clw = SW::lane_setup(p.conv, n0, p.n, wave, lane);
    typename SN::Lane cln{};
    if constexpr (NHWC) cln = SN::lane_setup(p.conv, n0, p.n, wave, lane);
    typename SNW::Lane clnw{};
    if constexpr (NHWCW) clnw = SNW::lane_setup(p.conv, n0, p.n, lane);
    auto issue_b = [&](float *lds, int k0) {
        if constexpr (NHWC)
            SN::issue(rb, lds, p.conv, cln, k0, kend, wave, lane);
        else if constexpr (NHWCW)
            SNW::issue(rb, lds, p.conv, clnw, k0, kend, wave);
        else if constexpr (CONVW)
            SW::issue(rb, gb, lds, p.conv, clw, k0, kend, wave, lane, wpatch);
        else if constexpr (CONVT)
            ST::issue(rb, lds, p.conv, n0, k0, p.n, kend, wave, lane);
        else if constexpr (CONV && GW == 16)
            SC16::issue(rb, gb, lds, p.conv, cl16, k0, kend, wave, lane, patch);
        else if constexpr (CONV)
            SC::issue(rb, lds, p.conv, cl, n0, k0, p.n, kend, wave, lane);
        else
            SB::issue(rb, lds, ldb, n0, k0, p.n, kend, wave, lane);
    };
    if (ktiles > 0) {
        SA::issue(ra, lds_a[0], lda, m0, kbeg, p.m, kend, wave, lane);
        issue_b(lds_b[0], kbeg);
    }
    for (int kt = 0; kt < ktiles; ++kt) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's part of slice kt is in LDS
        if constexpr (CONV && GW == 16) SC16::apply(lds_b[kt & 1], patch, wave, lane);
        if constexpr (CONVW) SW::apply(lds_b[kt & 1], wpatch, wave, lane);
        __syncthreads();  // every wave's part is; every wave is done reading slice kt - 1
        const int cur = kt & 1;
        if (kt + 1 < ktiles) {
            SA::issue(ra, lds_a[cur ^ 1], lda, m0, kbeg + (kt + 1) * BK, p.m, kend, wave, lane);
            issue_b(lds_b[cur ^ 1], kbeg + (kt + 1) * BK);
        }
        const float *la = lds_a[cur];
        const float *lb = lds_b[cur];
#pragma unroll
        for (int kg = 0; kg < BK; kg += 8) {
            float fa[FM][4], fb[FN][4];
            read_frags_dma<BM, BK, FM, AK>(la, wm0, kg, lane, fa);
            read_frags_dma<BN, BK, FN, BKC>(lb, wn0, kg, lane, fb);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn)
                        acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[fm][t], fb[fn][t], acc[fm][fn], 0, 0, 0);
        }
    }
    store_tile<BM, BN, WM, WN, AK, BKC>(p, acc, bz, m0, n0, wm0, wn0, lane, slice);
}

template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "6-bit vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait until at most `ahead` slices' loads (of kSliceLoads instructions
// each) are still in flight: vmcnt takes an immediate, so one branch per
// possible count.
template <int kSliceLoads, int NS>
__device__ __forceinline__ void vm_wait_slices(int ahead) {
    static_assert((NS - 1) * kSliceLoads < 64, "6-bit vmcnt");
    switch (ahead) {
    case 0: vm_wait<0>(); break;
    case 1: vm_wait<kSliceLoads>(); break;
    case 2: if constexpr (NS > 2) vm_wait<2 * kSliceLoads>(); break;
    case 3: if constexpr (NS > 3) vm_wait<3 * kSliceLoads>(); break;
    case 4: if constexpr (NS > 4) vm_wait<4 * kSliceLoads>(); break;
    case 5: if constexpr (NS > 5) vm_wait<5 * kSliceLoads>(); break;
    case 6: if constexpr (NS > 6) vm_wait<6 * kSliceLoads>(); break;
    default: if constexpr (NS > 7) vm_wait<7 * kSliceLoads>(); break;
    }
}

// The plain GEMM main loop with a fixed instruction schedule, for problems
// of about one round of tiles, where each SIMD holds one or two waves and
// every stall of a wave idles its matrix core.  Three LDS stages; slice
// kt + 2 is loaded while slice kt is multiplied.  The slice barrier sits
// before the last k group of a slice: the wave waits for its part of slice
// kt + 1, meets the others, refills the stage of slice kt - 1, reads the
// first fragments of slice kt + 1, and only then multiplies the last group
// of slice kt, whose fragments it read before the barrier.  Fragments are
// double-buffered across groups, and sched_barrier keeps the compiler from
// moving the LDS reads, the barrier or the DMA into the MFMA runs.  The
// barrier section runs in every iteration (the last one reads a stage it
// never uses), so the fragment waits of the last group see one set of
// pending reads.  Same K order per element as gemm_tile_dma, so the results
// are bit-identical to it.  On MI355X against gemm_tile_dma's two-stage
// loop: 4096x1024x1024 NT 76.4 -> 70.9 us (128x128, BK 32), 1024^3
// 26.0 -> 23.7 us (64x64, BK 32).
template <int BM, int BN, int BK, int WM, int WN, bool AK, bool BKC, int WA, int WB, int G = kGNone>
__device__ __forceinline__ void gemm_tile_pinned(const ZnGemmArgs &p, int wg = -1) {
    constexpr bool CONVT = G == kGTransposed, NHWC = G == kGNhwc, NHWCW = G == kGNhwcW;
    // gathers whose loads all go straight to LDS (no register-staged step)
    static_assert(G == kGNone || CONVT || NHWC || NHWCW, "gather not supported by the pinned loop");
    static_assert(!(CONVT || NHWC) || (BKC && WB == 16), "K-contiguous gathered operand");
    static_assert(!NHWCW || (!BKC && WB == 16), "X-contiguous gathered operand");
    constexpr int NT = WM * WN * kWave;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    constexpr int R = 3, GR = BK / 8;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
    static_assert(GR >= 2 && GR % 2 == 0, "an even number of k groups per slice");
    typedef DmaStage<BM, BK, NT, AK, WA> SA;
    typedef DmaStage<BN, BK, NT, BKC, WB> SB;  // the gathers issue as many loads per wave as SB
    typedef ConvTGatherStage<BN, BK, NT> ST;
    typedef ConvNhwcGatherStage<BN, BK, NT> SN;
    typedef ConvNhwcWGatherStage<BN, BK, NT> SNW;
    constexpr int L = SA::kPerWave + SB::kPerWave;  // DMA instructions per slice and wave
    __shared__ __attribute__((aligned(1024))) float lds_a[R][SA::kFloats];
    __shared__ __attribute__((aligned(1024))) float lds_b[R][SB::kFloats];

    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;
    int tm, tn, slice;
    tile_coords(p, tm, tn, slice, wg);
    const int m0 = tm * BM, n0 = tn * BN;
    const int64_t bz = blockIdx.y;

    const int kbeg = slice * p.k_chunk;
    const int kend = min(p.k, kbeg + p.k_chunk);
    const int ktiles = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int lda = (int)p.lda, ldb = (int)p.ldb;
    constexpr int RA = WA == 16 ? 3 : 0, RB = WB == 16 ? 3 : 0;
    const uint32_t a_bytes = (uint32_t)(AK ? (p.m - 1) * lda + ((p.k + RA) & ~RA) : (p.k - 1) * lda + ((p.m + RA) & ~RA)) * 4u;
    const uint32_t b_bytes =
        NHWCW ? (uint32_t)(p.conv.images * p.conv.channels * p.conv.in_h * p.conv.in_w) * 4u
        : (CONVT || NHWC) ? (uint32_t)(p.conv.channels * p.conv.in_h * p.conv.in_w) * 4u
                          : (uint32_t)(BKC ? (p.n - 1) * ldb + ((p.k + RB) & ~RB) : (p.k - 1) * ldb + ((p.n + RB) & ~RB)) * 4u;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + bz * p.stride_a, a_bytes);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b + bz * p.stride_b, b_bytes);
    typename SN::Lane cln{};
    if constexpr (NHWC) cln = SN::lane_setup(p.conv, n0, p.n, wave, lane);
    typename SNW::Lane clnw{};
    if constexpr (NHWCW) clnw = SNW::lane_setup(p.conv, n0, p.n, lane);
    // Plain 16-byte operands: each lane's DMA byte offsets at k = kbeg are
    // computed once per tile, masked on M and N; slice s adds s * inc, and K
    // is masked only in a partial last slice (an out-of-range offset plus
    // s * inc stays past the buffer's end, which is below 2^31 bytes).
    constexpr bool PRE = G == kGNone && WA == 16 && WB == 16;
    constexpr int LA = SA::kPerWave, LB = SB::kPerWave;
    uint32_t offa[LA], offb[LB];
    const uint32_t inca = (uint32_t)(AK ? BK : BK * lda) * 4u, incb = (uint32_t)(BKC ? BK : BK * ldb) * 4u;
    auto chunk = [&](int j, int kwaves, int per_inst) { return (j * kwaves + wave) * per_inst + 4 * lane; };
    if constexpr (PRE) {
#pragma unroll
        for (int j = 0; j < LA; ++j) {
            const int q = chunk(j, SA::kWaves, SA::kPerInst);
            const int outer = AK ? m0 + q / BK : kbeg + q / BM;
            const int inner = AK ? kbeg + 4 * (((q % BK) / 4) ^ SA::swz(q / BK)) : m0 + q % BM;
            offa[j] = (AK ? outer < p.m : inner < p.m) ? (uint32_t)(outer * lda + inner) * 4u : kOutOfRange;
        }
#pragma unroll
        for (int j = 0; j < LB; ++j) {
            const int q = chunk(j, SB::kWaves, SB::kPerInst);
            const int outer = BKC ? n0 + q / BK : kbeg + q / BN;
            const int inner = BKC ? kbeg + 4 * (((q % BK) / 4) ^ SB::swz(q / BK)) : n0 + q % BN;
            offb[j] = (BKC ? outer < p.n : inner < p.n) ? (uint32_t)(outer * ldb + inner) * 4u : kOutOfRange;
        }
    }
    const uint32_t lds_a0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(zn_lds_void *)&lds_a[0][0]);
    const uint32_t lds_b0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(zn_lds_void *)&lds_b[0][0]);
    auto issue = [&](int s, int st) {
        const int k0 = kbeg + s * BK;
        if constexpr (PRE) {
            const bool partial = k0 + BK > kend;
#pragma unroll
            for (int j = 0; j < LA; ++j) {
                uint32_t off = offa[j] + (uint32_t)s * inca;
                if (partial) {
                    const int q = chunk(j, SA::kWaves, SA::kPerInst);
                    const int kk = AK ? k0 + 4 * (((q % BK) / 4) ^ SA::swz(q / BK)) : k0 + q / BM;
                    if (kk >= kend) off = kOutOfRange;
                }
                const uint32_t dst = lds_a0 + (uint32_t)(st * SA::kFloats + (j * SA::kWaves + wave) * SA::kPerInst) * 4u;
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                             :
                             : "s"(dst), "v"(off), "s"(ra)
                             : "memory");
            }
#pragma unroll
            for (int j = 0; j < LB; ++j) {
                uint32_t off = offb[j] + (uint32_t)s * incb;
                if (partial) {
                    const int q = chunk(j, SB::kWaves, SB::kPerInst);
                    const int kk = BKC ? k0 + 4 * (((q % BK) / 4) ^ SB::swz(q / BK)) : k0 + q / BN;
                    if (kk >= kend) off = kOutOfRange;
                }
                const uint32_t dst = lds_b0 + (uint32_t)(st * SB::kFloats + (j * SB::kWaves + wave) * SB::kPerInst) * 4u;
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                             :
                             : "s"(dst), "v"(off), "s"(rb)
                             : "memory");
            }
            return;
        }
        SA::issue(ra, lds_a[st], lda, m0, k0, p.m, kend, wave, lane);
        if constexpr (NHWC)
            SN::issue(rb, lds_b[st], p.conv, cln, k0, kend, wave, lane);
        else if constexpr (NHWCW)
            SNW::issue(rb, lds_b[st], p.conv, clnw, k0, kend, wave);
        else if constexpr (CONVT)
            ST::issue(rb, lds_b[st], p.conv, n0, k0, p.n, kend, wave, lane);
        else
            SB::issue(rb, lds_b[st], ldb, n0, k0, p.n, kend, wave, lane);
    };

    zn_f32x16 acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0.0f;
    float fa[2][FM][4], fb[2][FN][4];
    auto multiply = [&](const float(&xa)[FM][4], const float(&xb)[FN][4]) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                for (int fn = 0; fn < FN; ++fn)
                    acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[fm][t], xb[fn][t], acc[fm][fn], 0, 0, 0);
    };
    if (ktiles > 0) {
        issue(0, 0);
        if (ktiles > 1) {
            issue(1, 1);
            vm_wait<L>();  // slice 0 is in; slice 1 may still be in flight
        } else {
            vm_wait<0>();
        }
        __syncthreads();
        read_frags_dma<BM, BK, FM, AK>(lds_a[0], wm0, 0, lane, fa[0]);
        read_frags_dma<BN, BK, FN, BKC>(lds_b[0], wn0, 0, lane, fb[0]);
    }
    int st = 0;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int nst = st + 1 == R ? 0 : st + 1;
#pragma unroll
        for (int g = 0; g + 1 < GR; ++g) {
            read_frags_dma<BM, BK, FM, AK>(lds_a[st], wm0, 8 * (g + 1), lane, fa[(g + 1) & 1]);
            read_frags_dma<BN, BK, FN, BKC>(lds_b[st], wn0, 8 * (g + 1), lane, fb[(g + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
            multiply(fa[g & 1], fb[g & 1]);
            __builtin_amdgcn_sched_barrier(0);
        }
        vm_wait<0>();     // this wave's part of slice kt + 1 is in LDS (the only DMA in flight)
        __syncthreads();  // every wave's part is; every wave is done with slice kt - 1
        if (kt + 2 < ktiles) issue(kt + 2, nst + 1 == R ? 0 : nst + 1);
        read_frags_dma<BM, BK, FM, AK>(lds_a[nst], wm0, 0, lane, fa[0]);
        read_frags_dma<BN, BK, FN, BKC>(lds_b[nst], wn0, 0, lane, fb[0]);
        __builtin_amdgcn_sched_barrier(0);
        multiply(fa[1], fb[1]);
        __builtin_amdgcn_sched_barrier(0);
        st = nst;
    }
    store_tile_fast<BM, BN, WM, WN, AK, BKC>(p, acc, bz, m0, n0, wm0, wn0, lane, slice);
}

// The main loop of the 256x256 tile (8 waves of 128x64) and of the 128x128
// tile with 16-byte rows (8 waves of 64x32): BK 16, 16-byte rows only, for
// problems of whole rounds of tiles; one workgroup per CU, two waves per
// SIMD, both held by the same barrier.  G = kGNhwcW gathers B from an NHWC
// batch (the convolution weight gradient, ConvNhwcWGatherStage's offsets).
//  * Operands are staged through registers, not LDS DMA: during k group 1
//    of slice kt every wave reads its share of slice kt + 2 (four 16-byte
//    buffer loads, into 16 registers; lanes out of range read zeros), and
//    during k group 0 of slice kt + 1 writes it into LDS, before the barrier
//    after which it is read.  Two LDS stages suffice: slice kt + 1 goes into
//    slice kt - 1's stage, which no wave has read since the previous
//    barrier.  MI355X, 8192^3, against the same loop fed by LDS DMA (three
//    stages, one wave per SIMD issuing a slice as one burst): NN 146.0 ->
//    149.7, NT 147.2 -> 149.8, TN 144.2 -> 150.5 TFLOP/s.  With its DMA
//    removed the DMA loop ran at 151.5 (NN), so the DMA cost 3.7%; neither
//    its latency (a fourth stage lost 1.4%) nor the barrier (removed: no
//    change) was the cause.  Loading during k group 0 as well was 1% slower,
//    and one loading wave per SIMD with twice the share 30% slower.
//  * The LDS reads of the next k group are issued one at a time between the
//    MFMAs of the current one, rather than as a burst before them.  A burst
//    of a workgroup's 8 waves filled the CU's LDS command queue, and a wave
//    whose read cannot issue stalls its later MFMAs (SQ_LDS_CMD_FIFO_FULL:
//    2e7 -> 0 cycles; 8192^3 NN on 4 waves of 128x128: 137.5 -> 141.4
//    TFLOP/s).  The loads and LDS writes take the MFMA runs after the reads;
//    where a group has fewer runs than reads plus loads (the 128x128 tile:
//    8 runs), the last runs carry a read and a load or write each.  On the
//    128x128 tile against the pinned loop: 4096x1024x1024 NT 70.0 -> 66.0
//    us, 2048^3 NN 133.1 -> 129.6 us.
//  * Each lane's load offsets are computed once per tile (masked on M and
//    N); slice s adds s times an increment, and a load whose k lies at or
//    beyond the end of K reads zeros, without branches.
// Each element sums K in the same order as the other tiles, so results are
// bit-identical to them.
//  * UA (the _u kernels): rows that are not whole float4s, loaded as they
//    lie with 16-byte loads at 4-byte aligned offsets, which gfx950 serves.
//    Each buffer spans the operand exactly; the range check is per dword,
//    so a load that runs past the end returns zeros for the dwords beyond
//    it and the data before it.  A load of an X-contiguous operand that
//    runs past X reads the next row's first values into columns (or rows)
//    of C that are never stored.  A load of a K-contiguous operand that
//    runs past K reads the next row's first values as k >= K: those are set
//    to zero in registers before the LDS write (an Inf or NaN there would
//    otherwise reach C through a product with a zero).
template <int BM, int BN, int BK, int WM, int WN, bool AK, bool BKC, int G = kGNone, bool UA = false>
__device__ __forceinline__ void gemm_tile_wide(const ZnGemmArgs &p, int wg = -1) {
    constexpr int NT = WM * WN * kWave;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    static_assert(BK == 16, "two k groups per slice");
    constexpr bool NHWCW = G == kGNhwcW;  // B gathered from an NHWC batch (convolution weight gradient)
    static_assert(G == kGNone || (NHWCW && !BKC), "the NHWC weight-gradient gather only, X-contiguous");
    typedef ConvNhwcWGatherStage<BN, BK, NT> SNW;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
    typedef DmaStage<BM, BK, NT, AK, 16> SA;  // the LDS layout of the DMA loops
    typedef DmaStage<BN, BK, NT, BKC, 16> SB;
    constexpr int LA = SA::kPerWave, LB = SB::kPerWave, L = LA + LB;  // 16-byte loads per slice and wave
    constexpr int RA = AK ? FM : 4, RB = BKC ? FN : 4, NR = RA + RB;  // LDS reads per k group
    // the runs after which a load or LDS write goes: after the reads when
    // there is room (the 256x256 tile), else the last L runs, after a read
    constexpr int kX0 = NR + L <= 4 * FM ? NR : 4 * FM - L;
    static_assert(NR <= 4 * FM && kX0 >= 0, "at most one read and one load or write after each (t, fm) MFMA run");
    __shared__ __attribute__((aligned(1024))) float lds_a[2][SA::kFloats];
    __shared__ __attribute__((aligned(1024))) float lds_b[2][SB::kFloats];

    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;
    int tm, tn, slice;
    tile_coords(p, tm, tn, slice, wg);
    const int m0 = tm * BM, n0 = tn * BN;
    const int64_t bz = blockIdx.y;
    const int kbeg = slice * p.k_chunk;
    const int kend = min(p.k, kbeg + p.k_chunk);
    const int ktiles = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int lda = (int)p.lda, ldb = (int)p.ldb;
    static_assert(!(UA && NHWCW), "unaligned rows: plain operands only");
    static_assert(!UA || NT == 512, "the folded row tail covers K <= 2 * 512 (the host's bound)");
    constexpr int RU = UA ? 0 : 3;  // whole float4 rows are padded to a multiple of 4 (packed copies)
    const uint32_t a_bytes = (uint32_t)(AK ? (p.m - 1) * lda + ((p.k + RU) & ~RU) : (p.k - 1) * lda + ((p.m + RU) & ~RU)) * 4u;
    const uint32_t b_bytes = NHWCW ? (uint32_t)(p.conv.images * p.conv.channels * p.conv.in_h * p.conv.in_w) * 4u
                                   : (uint32_t)(BKC ? (p.n - 1) * ldb + ((p.k + RU) & ~RU) : (p.k - 1) * ldb + ((p.n + RU) & ~RU)) * 4u;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + bz * p.stride_a, a_bytes);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b + bz * p.stride_b, b_bytes);

    // This lane's loads at k = kbeg, as byte offsets masked on M and N, and
    // the k offset of each within a slice: slice s adds s * inc, and a load
    // whose k falls at or beyond kend reads zeros.  No branches: the loads
    // past the last slice read zeros into registers nobody writes out.
    auto chunk = [&](int j, int kwaves, int per_inst) { return (j * kwaves + wave) * per_inst + 4 * lane; };
    uint32_t off0[L], inc[L];
    int kq[L];
#pragma unroll
    for (int j = 0; j < LA; ++j) {
        const int q = chunk(j, SA::kWaves, SA::kPerInst);
        kq[j] = AK ? 4 * (((q % BK) / 4) ^ SA::swz(q / BK)) : q / BM;
        const int outer = AK ? m0 + q / BK : kbeg + q / BM;
        const int inner = AK ? kbeg + kq[j] : m0 + q % BM;
        off0[j] = (AK ? outer < p.m : inner < p.m) ? (uint32_t)(outer * lda + inner) * 4u : kOutOfRange;
        inc[j] = (uint32_t)(AK ? BK : BK * lda) * 4u;
    }
#pragma unroll
    for (int j = 0; j < LB; ++j) {
        const int q = chunk(j, SB::kWaves, SB::kPerInst);
        kq[LA + j] = BKC ? 4 * (((q % BK) / 4) ^ SB::swz(q / BK)) : q / BN;
        const int outer = BKC ? n0 + q / BK : kbeg + q / BN;
        const int inner = BKC ? kbeg + kq[LA + j] : n0 + q % BN;
        off0[LA + j] = (BKC ? outer < p.n : inner < p.n) ? (uint32_t)(outer * ldb + inner) * 4u : kOutOfRange;
        inc[LA + j] = (uint32_t)(BKC ? BK : BK * ldb) * 4u;
    }
    const int klen = kend - kbeg;
    typename SNW::Lane clnw{};
    if constexpr (NHWCW) clnw = SNW::lane_setup(p.conv, n0, p.n, lane);
    zn_f32x4 g[L];  // this wave's share of one slice
    auto load = [&](int s, int j) {
        uint32_t off = s * BK + kq[j] < klen && off0[j] != kOutOfRange ? off0[j] + (uint32_t)s * inc[j] : kOutOfRange;
        if (NHWCW && j >= LA) off = SNW::offset(p.conv, clnw, kbeg + s * BK, kend, wave, j - LA);
        g[j] = __builtin_bit_cast(zn_f32x4, __builtin_amdgcn_raw_buffer_load_b128(j < LA ? ra : rb, off, 0, 0));
    };
    // write load j of slice s into stage st
    auto write = [&](int st, int j, int s) {
        zn_f32x4 v = g[j];
        if constexpr (UA) {
            if ((AK && j < LA) || (BKC && j >= LA)) {  // K-contiguous: zero the values at k >= kend
                const int rem = klen - (s * BK + kq[j]);
#pragma unroll
                for (int e = 1; e < 4; ++e) v[e] = e < rem ? v[e] : 0.0f;
            }
        }
        if (j < LA)
            *reinterpret_cast<zn_f32x4 *>(&lds_a[st][chunk(j, SA::kWaves, SA::kPerInst)]) = v;
        else
            *reinterpret_cast<zn_f32x4 *>(&lds_b[st][chunk(j - LA, SB::kWaves, SB::kPerInst)]) = v;
    };

    // Row tail (UA kernels, p.tail_rows > 0): this workgroup's tail elements
    // o = w * P + q, q < P <= 4, each over K <= 1024: thread tid multiplies
    // k = tid and k = tid + NT.  Its operands are loaded here, before the
    // main loop, so that their latency hides behind it; the products and
    // the sums come after it.
    float tail_av[4][2], tail_bv[4][2];
    int tail_t[4], tail_j[4];
    const bool has_tail = UA && p.tail_rows > 0;  // uniform
    if constexpr (UA) {
        if (has_tail) {
            const int P = p.tail_per_wg;
            const int total = p.tail_rows * p.n;
            const int o0 = (int)(blockIdx.x + gridDim.x * blockIdx.z) * P;
            int t = o0 / p.n, j = o0 - t * p.n;
            const __amdgpu_buffer_rsrc_t rt = make_rsrc(
                p.tail_a, (uint32_t)(AK ? (p.tail_rows - 1) * lda + p.k : (p.k - 1) * lda + p.tail_rows) * 4u);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                tail_t[q] = t;
                tail_j[q] = j;
                const bool ok = q < P && o0 + q < total;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int k = tid + i * NT;
                    const bool in = ok && k < p.k;
                    const int ao = AK ? t * lda + k : k * lda + t;
                    const int bo = BKC ? j * ldb + k : k * ldb + j;
                    tail_av[q][i] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(rt, in ? (uint32_t)ao * 4u : kOutOfRange, 0, 0));
                    tail_bv[q][i] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(rb, in ? (uint32_t)bo * 4u : kOutOfRange, 0, 0));
                }
                if (++j == p.n) {
                    j = 0;
                    ++t;
                }
            }
        }
    }

    zn_f32x16 acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0.0f;
    float fa[2][FM][4], fb[2][FN][4];
    // One k group from fragments (xa, xb); after MFMA run q (one (t, fm)
    // pair, FN MFMAs): q < NR reads fragment q of the next group from stage
    // rst at k rkg, and q >= kX0 calls `extra(q - kX0)` (a load or an LDS
    // write).
    auto multiply = [&](const float(&xa)[FM][4], const float(&xb)[FN][4], int rst, int rkg, float(&da)[FM][4],
                        float(&db)[FN][4], auto &&extra) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
                for (int fn = 0; fn < FN; ++fn)
                    acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[fm][t], xb[fn][t], acc[fm][fn], 0, 0, 0);
                const int q = t * FM + fm;
                __builtin_amdgcn_sched_barrier(0);
                if (q < NR) {
                    if (q < RA)
                        read_frag_one<BM, BK, FM, AK>(lds_a[rst], wm0, rkg, lane, q, da);
                    else
                        read_frag_one<BN, BK, FN, BKC>(lds_b[rst], wn0, rkg, lane, q - RA, db);
                }
                if (q >= kX0) extra(q - kX0);
                __builtin_amdgcn_sched_barrier(0);
            }
    };
    // Slice kt in stage S = kt % 2: group 0 writes slice kt + 1 (in the
    // registers since group 1 of slice kt - 1) into stage S ^ 1, the barrier,
    // group 1 loads slice kt + 2 while reading slice kt + 1's group 0.
    auto slice_step = [&](int kt, auto sc) {
        constexpr int S = decltype(sc)::value;
        auto wr = [&](int x) {
            if (x < L) write(S ^ 1, x, kt + 1);
        };
        auto ld = [&](int x) {
            if (x < L) load(kt + 2, x);
        };
        multiply(fa[0], fb[0], S, 8, fa[1], fb[1], wr);  // group 0; reads group 1
        __syncthreads();  // slice kt + 1 is in LDS; every wave has read slice kt for the last time
        __builtin_amdgcn_sched_barrier(0);
        multiply(fa[1], fb[1], S ^ 1, 0, fa[0], fb[0], ld);  // group 1; reads group 0 of slice kt + 1
        __builtin_amdgcn_sched_barrier(0);
    };
    if (ktiles > 0) {
#pragma unroll
        for (int j = 0; j < L; ++j) load(0, j);
#pragma unroll
        for (int j = 0; j < L; ++j) write(0, j, 0);
#pragma unroll
        for (int j = 0; j < L; ++j) load(1, j);
        __syncthreads();
        read_frags_dma<BM, BK, FM, AK>(lds_a[0], wm0, 0, lane, fa[0]);
        read_frags_dma<BN, BK, FN, BKC>(lds_b[0], wn0, 0, lane, fb[0]);
    }
    for (int kt = 0; kt < ktiles; kt += 2) {
        slice_step(kt, std::integral_constant<int, 0>());
        if (kt + 1 < ktiles) slice_step(kt + 1, std::integral_constant<int, 1>());
    }
    if constexpr (UA) {
        if (has_tail) {
            // each thread's products (k ascending), the wave's sum over a fixed
            // butterfly read from lane 0, then the waves' sums in wave order
            __shared__ float tail_red[4][NT / kWave];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float v = tail_av[q][0] * tail_bv[q][0];
                v = v + tail_av[q][1] * tail_bv[q][1];
#pragma unroll
                for (int off = kWave / 2; off > 0; off >>= 1) v = v + __shfl_xor(v, off, kWave);
                if (lane == 0) tail_red[q][wave] = v;
            }
            __syncthreads();
            const int P = p.tail_per_wg;
            const int o0 = (int)(blockIdx.x + gridDim.x * blockIdx.z) * P;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (tid == q && q < P && o0 + q < p.tail_rows * p.n) {
                    float v = tail_red[q][0];
#pragma unroll
                    for (int w = 1; w < NT / kWave; ++w) v = v + tail_red[q][w];
                    float *dst = p.tail_c + (int64_t)tail_t[q] * p.ldc + tail_j[q];
                    if (p.accumulate) v = *dst + v;
                    if (p.bias) v = v + p.bias[p.bias_rows ? p.m + tail_t[q] : tail_j[q]];
                    *dst = zn_activate(v, p.act);
                }
            }
        }
    }
    store_tile_fast<BM, BN, WM, WN, AK, BKC>(p, acc, bz, m0, n0, wm0, wn0, lane, slice);
}

// The end of an intra-workgroup split-K tile (gemm_ksplit and the fused
// Dense backward tile): the KS partial BM x BN tiles go to LDS (which the
// staging no longer uses), each output is the sum of its partials in wave
// order, and the epilogue applies C_old, the bias and the activation; wave w
// finishes the (row block, register) items w, w + KS, ...
//
// XS (the zn_sgemmk4s_* kernels): the workgroups split K as well; wave w of
// workgroup s multiplied K slice q = s * KS + w, each non-empty slice's
// partial tile goes to its own block of p.ws, and the workgroup that arrives
// last at the tile's counter (whichever it is) adds the blocks in slice
// order, runs the epilogue and sets the counter back to zero.  The blocks
// are written and read as agent-scope atomics (stores and loads coherent
// across the XCDs' L2 caches), and every store has completed (vmcnt 0)
// before the workgroup arrives, so the last arrival reads finished blocks.
// Device-scope fences would write back and invalidate a whole L2 per
// workgroup instead (36 us against 14 us for 224 workgroups on MI355X).
// Kept out of the other kernels: in C2's small launches the unused code
// alone cost about 2 us per launch.
template <int BM, int BN, int KS, bool AK, bool BKC, int ACT, bool XS = false>
__device__ __forceinline__ void ksplit_finish(const ZnGemmArgs &p, float *lds,
                                              const zn_f32x16 (&acc)[BM / 32][BN / 32], int64_t bz, int m0, int n0,
                                              int wave, int lane, int tile = 0, int split = 0) {
    constexpr int FM = BM / 32, FN = BN / 32;
    int slices = KS;
    float *src = lds;
    if constexpr (XS) {
        constexpr int kWavePart = FM * FN * 16 * kWave;
        slices = (p.k + p.k_chunk - 1) / p.k_chunk;
        const int64_t slot = bz * ((int64_t)p.tiles_m * p.tiles_n) + tile;
        src = p.ws + slot * p.splits * KS * kWavePart;
        const int q = split * KS + wave;
        if (q < slices) {
            float *mine = src + (int64_t)q * kWavePart;
#pragma unroll
            for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        __hip_atomic_store(mine + ((fm * FN + fn) * 16 + r) * kWave + lane, acc[fm][fn][r],
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __shared__ int last;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's block is written
        __syncthreads();
        if (threadIdx.x == 0)
            last = __hip_atomic_fetch_add(p.counters + slot * kCounterStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   p.splits - 1;
        __syncthreads();
        if (!last) return;
        if (threadIdx.x == 0) __hip_atomic_store(p.counters + slot * kCounterStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        // partial tiles to LDS: part[wave][fm][fn][r][lane], lanes contiguous
        __syncthreads();  // every wave is done with every staging region
        float *part = lds + wave * (FM * FN * 16 * kWave);
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                for (int r = 0; r < 16; ++r) part[((fm * FN + fn) * 16 + r) * kWave + lane] = acc[fm][fn][r];
        __syncthreads();
    }

    float *gc = p.c + bz * p.stride_c;
    const int64_t ldc = p.ldc;
    const int j = lane & 31, h = lane >> 5;
    const bool has_bias = p.bias != nullptr;
    const bool vec = !BKC && FN > 1 && p.vec_c != 0;
    constexpr int kPart = FM * FN * 16 * kWave;
    for (int item = wave; item < FM * 16; item += KS) {
        const int fm = item >> 4, r = item & 15;
        const int bi = 8 * (r >> 2) + 4 * h + (r & 3);
        const int row = m0 + (AK ? 32 * fm + bi : FM * bi + fm);
        if (row >= p.m) continue;
        float *crow = gc + (int64_t)row * ldc;
        const float rbias = has_bias && p.bias_rows ? p.bias[row] : 0.0f;
        float v[FN];
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
            const int off = ((fm * FN + fn) * 16 + r) * kWave + lane;
            float x;
            if constexpr (XS) {
                // in groups of 16 loads, so the loads of a group are in flight together
                x = __hip_atomic_load(src + off, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                for (int q0 = 1; q0 < slices; q0 += 16) {
                    float t[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        t[i] = q0 + i < slices ? __hip_atomic_load(src + (int64_t)(q0 + i) * kPart + off,
                                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                               : 0.0f;
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (q0 + i < slices) x = x + t[i];
                }
            } else {
                x = lds[off];
#pragma unroll
                for (int w = 1; w < KS; ++w) x = x + lds[w * kPart + off];
            }
            v[fn] = x;
        }
        if constexpr (!BKC && FN > 1) {
            const int col0 = n0 + FN * j;
            if (vec && col0 + FN <= p.n && !p.chain_gaa) {  // a chained derivative takes the scalar path
                typedef typename FVec<FN>::type VT;
                VT *dst = reinterpret_cast<VT *>(crow + col0);
                VT o;
                if (p.accumulate) o = *dst;
#pragma unroll
                for (int fn = 0; fn < FN; ++fn) {
                    float x = v[fn];
                    if (p.accumulate) x = o[fn] + x;
                    if (has_bias) x = x + (p.bias_rows ? rbias : p.bias[col0 + fn]);
                    o[fn] = zn_activate(x, ACT);
                }
                *dst = o;
                continue;
            }
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
            const int col = n0 + (BKC ? 32 * fn + j : FN * j + fn);
            if (col >= p.n) continue;
            float x = v[fn];
            if (p.accumulate) x = crow[col] + x;
            if (has_bias) x = x + (p.bias_rows ? rbias : p.bias[col]);
            x = zn_activate(x, ACT);
            crow[col] = x;
            if (p.chain_gaa) {
                const int64_t at = (int64_t)row * ldc + col;
                p.chain_gaa[at] = zn_act_backward(p.chain_y[at], x, p.chain_act);
            }
        }
    }
}

// Intra-workgroup split-K, for problems of few tiles and long K: each of the
// KS waves of a workgroup multiplies the whole BM x BN tile over its own
// contiguous range of K (the ranges of a K split into KS slices of whole BK
// multiples), staging its operands by DMA into two private LDS stages, so
// the main loop has no barrier: a wave waits only for its own loads.  The
// partial tiles then meet in LDS and are summed in wave order, 0 to KS - 1,
// as the split-K reduce sums its slices (deterministic), and the epilogue
// (C_old, bias, activation) runs on the sums; wave w finishes the (row
// block, register) items w, w + KS, ...  No workspace, no second launch.
//
// `lds` holds KS private regions of two A and two B stages each
// (KS * 2 * (BM + BN) * BK floats); the partial tiles reuse it.
//
// XS: K is split over workgroups too (blockIdx.z = split of p.splits): wave
// w of workgroup s takes slice s * KS + w of p.k_chunk, and ksplit_finish
// hands the partial tiles over through p.ws.  PF (with XS): both stages
// are filled before the first wait, so a wave of one or two slices waits
// for one memory round trip.  (In C2's small launches that prologue
// measured 1.5 us slower per launch, and C1's 512^3 0.07 us faster.)
template <int BM, int BN, int BK, int KS, bool AK, bool BKC, int WA, int WB, int ACT, bool XS = false, bool PF = XS>
__device__ __forceinline__ void gemm_ksplit(const ZnGemmArgs &p, float *lds, int wg = -1) {
    constexpr int FM = BM / 32, FN = BN / 32;
    typedef DmaStage<BM, BK, kWave, AK, WA> SA;
    typedef DmaStage<BN, BK, kWave, BKC, WB> SB;
    constexpr int kRegion = 2 * (SA::kFloats + SB::kFloats);
    static_assert(FM * FN * 16 * kWave <= kRegion, "a wave's partial tile fits in its staging region");
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
    // Stage s of A and of B: offsets from the LDS array itself (a pointer
    // picked from an array of pointers at run time loses its address space,
    // and the fragment reads became flat loads that also wait for the DMA).
    float *const region = lds + wave * kRegion;
    auto stage_a = [region](int s) { return region + s * SA::kFloats; };
    auto stage_b = [region](int s) { return region + 2 * SA::kFloats + s * SB::kFloats; };

    const int pid = wg >= 0 ? wg : (int)blockIdx.x;  // wg >= 0: this workgroup's tile in a grouped launch
    const int tm = pid / p.tiles_n, tn = pid - tm * p.tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;
    const int64_t bz = wg >= 0 ? 0 : blockIdx.y;
    const int split = XS ? (int)blockIdx.z : 0;
    const int chunk = XS ? p.k_chunk : ((p.k + KS - 1) / KS + BK - 1) / BK * BK;
    const int kbeg = min(p.k, (split * KS + wave) * chunk);
    const int kend = min(p.k, kbeg + chunk);
    const int ktiles = (kend - kbeg + BK - 1) / BK;
    const int lda = (int)p.lda, ldb = (int)p.ldb;
    constexpr int RA = WA == 16 ? 3 : 0, RB = WB == 16 ? 3 : 0;
    const uint32_t a_bytes = (uint32_t)(AK ? (p.m - 1) * lda + ((p.k + RA) & ~RA) : (p.k - 1) * lda + ((p.m + RA) & ~RA)) * 4u;
    const uint32_t b_bytes = (uint32_t)(BKC ? (p.n - 1) * ldb + ((p.k + RB) & ~RB) : (p.k - 1) * ldb + ((p.n + RB) & ~RB)) * 4u;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + bz * p.stride_a, a_bytes);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b + bz * p.stride_b, b_bytes);

    zn_f32x16 acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0.0f;
    constexpr int kSliceLoads = SA::kPerWave + SB::kPerWave;  // this wave's load instructions per slice
    for (int kt = 0; kt < (PF ? 2 : 1) && kt < ktiles; ++kt) {
        SA::issue(ra, stage_a(kt), lda, m0, kbeg + kt * BK, p.m, kend, 0, lane);
        SB::issue(rb, stage_b(kt), ldb, n0, kbeg + kt * BK, p.n, kend, 0, lane);
    }
    for (int kt = 0; kt < ktiles; ++kt) {
        const int cur = kt & 1;
        if constexpr (PF) {
            if (kt + 1 < ktiles)
                vm_wait<kSliceLoads>();  // slice kt is in its stage; slice kt + 1 may still be in flight
            else
                vm_wait<0>();
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // slice kt is in this wave's stage
            if (kt + 1 < ktiles) {  // the other stage was last read by slice kt - 1, whose MFMAs consumed those reads
                SA::issue(ra, stage_a(cur ^ 1), lda, m0, kbeg + (kt + 1) * BK, p.m, kend, 0, lane);
                SB::issue(rb, stage_b(cur ^ 1), ldb, n0, kbeg + (kt + 1) * BK, p.n, kend, 0, lane);
            }
        }
#pragma unroll
        for (int kg = 0; kg < BK; kg += 8) {
            float fa[FM][4], fb[FN][4];
            read_frags_dma<BM, BK, FM, AK>(stage_a(cur), 0, kg, lane, fa);
            read_frags_dma<BN, BK, FN, BKC>(stage_b(cur), 0, kg, lane, fb);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn)
                        acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[fm][t], fb[fn][t], acc[fm][fn], 0, 0, 0);
        }
        if (PF && kt + 2 < ktiles) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this stage's fragment reads have returned
            SA::issue(ra, stage_a(cur), lda, m0, kbeg + (kt + 2) * BK, p.m, kend, 0, lane);
            SB::issue(rb, stage_b(cur), ldb, n0, kbeg + (kt + 2) * BK, p.n, kend, 0, lane);
        }
    }

    ksplit_finish<BM, BN, KS, AK, BKC, ACT, XS>(p, lds, acc, bz, m0, n0, wave, lane, pid, split);
}

// Intra-workgroup split-K on 16x16 tiles (v_mfma_f32_16x16x4f32), for
// problems whose 32x32 tiles would leave most CUs idle: C2's 256 x 128 x 784
// forward is 32 tiles of 32x32 (at least 2.6 us of matrix-core time on each
// of 32 CUs) but 128 tiles of 16x16.  Each of the KS = 4 waves multiplies
// the 16x16 tile over its own contiguous range of K (whole BK = 32 slices),
// with up to NS slices in flight in NS private LDS stages (8 with 16-byte
// loads: every slice of a wave of up to 8 slices is requested before the
// first wait), then the partial tiles meet in LDS and are added in wave
// order, and the epilogue (C_old, bias, activation) runs on the sums.
//
// 16x16x4 operands: in MFMA step t of a k group kg (16 values of k), lane
// (i = lane % 16, h = lane / 16) supplies A[i][kg + 4h + t] and
// B[kg + 4h + t][i]; lane (j, h) receives D[4h + r][j] in register r.
// `lds` holds KS * NS stages of (16 + 16) * BK floats.  NSMAX = 2 (the
// zn_sgemmq4m_* kernels): two stages, 32 KB of LDS, so that five
// workgroups share a CU when there are more tiles than CUs.
// gemm_ksplit16 up to the epilogue: returns the sum (in wave order) of the
// KS partial values of tile element (threadIdx.x / 16, threadIdx.x % 16).
//
// KS = 8 or 16 (the two-layer forward): two or four waves per SIMD, and K's
// slices dealt out as evenly as whole slices allow (wave w takes slices
// [w S / KS, (w + 1) S / KS) of S); threads 0..255 return the sums.
template <int KS, bool AK, bool BKC, int W, int NSMAX = 8>
__device__ __forceinline__ float gemm_ksplit16_sum(const ZnGemmArgs &p, float *lds, int m0, int n0, int64_t bz) {
    constexpr int BM = 16, BN = 16, BK = 32;
    constexpr int NS = NSMAX < (W == 16 ? 8 : 4) ? NSMAX : (W == 16 ? 8 : 4);
    typedef DmaStage<BM, BK, kWave, AK, W> SA;
    typedef DmaStage<BN, BK, kWave, BKC, W> SB;
    constexpr int kStage = SA::kFloats + SB::kFloats;
    constexpr int kSliceLoads = SA::kPerWave + SB::kPerWave;
    static_assert(KS == 4 || KS == 8 || KS == 16, "4, 8 or 16 waves; threads 0..255 finish one output element each");
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
    float *region = lds + wave * NS * kStage;

    int kbeg, kend;
    if constexpr (KS > 4) {
        const int slices = (p.k + BK - 1) / BK;
        kbeg = min(p.k, wave * slices / KS * BK);
        kend = min(p.k, (wave + 1) * slices / KS * BK);
    } else {
        const int chunk = ((p.k + KS - 1) / KS + BK - 1) / BK * BK;
        kbeg = min(p.k, wave * chunk);
        kend = min(p.k, kbeg + chunk);
    }
    const int ktiles = (kend - kbeg + BK - 1) / BK;
    const int lda = (int)p.lda, ldb = (int)p.ldb;
    constexpr int RW = W == 16 ? 3 : 0;
    const uint32_t a_bytes = (uint32_t)(AK ? (p.m - 1) * lda + ((p.k + RW) & ~RW) : (p.k - 1) * lda + ((p.m + RW) & ~RW)) * 4u;
    const uint32_t b_bytes = (uint32_t)(BKC ? (p.n - 1) * ldb + ((p.k + RW) & ~RW) : (p.k - 1) * ldb + ((p.n + RW) & ~RW)) * 4u;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + bz * p.stride_a, a_bytes);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b + bz * p.stride_b, b_bytes);

    for (int kt = 0; kt < NS && kt < ktiles; ++kt) {
        float *st = region + kt * kStage;
        SA::issue(ra, st, lda, m0, kbeg + kt * BK, p.m, kend, 0, lane);
        SB::issue(rb, st + SA::kFloats, ldb, n0, kbeg + kt * BK, p.n, kend, 0, lane);
    }
    const int i = lane & 15, h = lane >> 4;
    zn_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int kt = 0; kt < ktiles; ++kt) {
        vm_wait_slices<kSliceLoads, NS>(min(ktiles - 1 - kt, NS - 1));  // slice kt is in its stage
        const float *sa = region + (kt % NS) * kStage;
        const float *sb = sa + SA::kFloats;
#pragma unroll
        for (int kg = 0; kg < BK; kg += 16) {
            float fa[4], fb[4];
            if constexpr (AK) {
                const int slot = (kg / 4 + h) ^ SA::swz(i);
                const zn_f32x4 v = *reinterpret_cast<const zn_f32x4 *>(sa + i * BK + 4 * slot);
#pragma unroll
                for (int t = 0; t < 4; ++t) fa[t] = v[t];
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) fa[t] = sa[(kg + 4 * h + t) * BM + i];
            }
            if constexpr (BKC) {
                const int slot = (kg / 4 + h) ^ SB::swz(i);
                const zn_f32x4 v = *reinterpret_cast<const zn_f32x4 *>(sb + i * BK + 4 * slot);
#pragma unroll
                for (int t = 0; t < 4; ++t) fb[t] = v[t];
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) fb[t] = sb[(kg + 4 * h + t) * BN + i];
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[t], fb[t], acc, 0, 0, 0);
        }
        if (kt + NS < ktiles) {  // refill this stage once its fragment reads have returned
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            float *st = region + (kt % NS) * kStage;
            SA::issue(ra, st, lda, m0, kbeg + (kt + NS) * BK, p.m, kend, 0, lane);
            SB::issue(rb, st + SA::kFloats, ldb, n0, kbeg + (kt + NS) * BK, p.n, kend, 0, lane);
        }
    }

    // partial tiles to LDS, part[wave][r][lane]; thread t finishes element
    // (t / 16, t % 16), held by lane 16 * (t / 64) + t % 16 in register (t / 16) % 4
    __syncthreads();  // every wave is done with every stage
    float *part = lds + wave * 4 * kWave;
#pragma unroll
    for (int r = 0; r < 4; ++r) part[r * kWave + lane] = acc[r];
    __syncthreads();
    const int t = threadIdx.x & 255;
    const int rr = t >> 4, cc = t & 15;
    const int off = (rr & 3) * kWave + (rr >> 2) * 16 + cc;
    float x = lds[off];
#pragma unroll
    for (int w = 1; w < KS; ++w) x = x + lds[w * 4 * kWave + off];
    return x;
}

template <int KS, bool AK, bool BKC, int W, int ACT, int NSMAX = 8>
__device__ __forceinline__ void gemm_ksplit16(const ZnGemmArgs &p, float *lds) {
    const int pid = blockIdx.x;
    const int tm = pid / p.tiles_n, tn = pid - tm * p.tiles_n;
    const int m0 = tm * 16, n0 = tn * 16;
    const int64_t bz = blockIdx.y;
    float x = gemm_ksplit16_sum<KS, AK, BKC, W, NSMAX>(p, lds, m0, n0, bz);
    if (threadIdx.x >= 256) return;  // eight waves: threads 0..255 own the elements
    const int t = threadIdx.x;
    const int row = m0 + (t >> 4), col = n0 + (t & 15);
    if (row < p.m && col < p.n) {
        float *dst = p.c + bz * p.stride_c + (int64_t)row * p.ldc + col;
        if (p.accumulate) x = *dst + x;
        if (p.bias) x = x + p.bias[p.bias_rows ? row : col];
        *dst = zn_activate(x, ACT);
    }
}

// Store instructions a wave issues for a tile that lies wholly inside C:
// one per (row block, accumulator register) on the vector-store path of an
// X-contiguous B, one per element column otherwise (fewest of the two, since
// vec_c decides at run time).  Capped at the 6-bit vmcnt field.
template <int FM, int FN, bool BKC>
constexpr int interior_stores() {
    return (!BKC && FN > 1 ? FM * 16 : FM * 16 * FN) < 63 ? (!BKC && FN > 1 ? FM * 16 : FM * 16 * FN) : 63;
}

// Persistent plain GEMM (unsplit, one or more problems): workgroup g takes
// the work items g, g + G, g + 2G, ... (G = gridDim.x) of the problem-major,
// row-major (problem, tile) order, and the two-stage LDS pipeline runs on
// across tile boundaries: the first slice of the next tile is in flight
// while the last slice of the current one is multiplied and its results are
// stored, so no tile waits for its first load or a fresh dispatch.  The
// activation is a template argument (the kernel dispatches once at entry).
//
// The first wait of a tile must cover that prefetch but not the stores
// issued after it.  Vector memory operations of a wave retire in issue order
// (the compiler's own waits rely on it: a load followed by two stores is
// awaited with vmcnt(2)), so after a tile that lay wholly inside C, whose
// epilogue issued at least S = interior_stores() stores after the prefetch,
// vmcnt(S) leaves only those stores in flight; after an edge tile (fewer
// stores) it waits for everything.
//
// These problems are bound by writing C (C5 QK^T: K = 64, 512 MiB of C, at
// 2 * 64 flops per 4 bytes written), so C goes out with non-temporal stores:
// on MI355X that took the QK^T batch from 217 to 201 us.  The same stores in
// the other kernels changed nothing beyond run-to-run noise.
// `lds` holds the two A stages, then the two B stages (2 * (BM + BN) * BK
// floats, 1 KB aligned), declared by the kernel once for all activations.
template <int BM, int BN, int BK, int WM, int WN, bool AK, bool BKC, int WA, int WB, int ACT>
__device__ __forceinline__ void gemm_persistent(const ZnGemmArgs &p, float *lds) {
    constexpr int NT = WM * WN * kWave;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    constexpr int S = interior_stores<FM, FN, BKC>();
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
    typedef DmaStage<BM, BK, NT, AK, WA> SA;
    typedef DmaStage<BN, BK, NT, BKC, WB> SB;
    float(*lds_a)[SA::kFloats] = reinterpret_cast<float(*)[SA::kFloats]>(lds);
    float(*lds_b)[SB::kFloats] = reinterpret_cast<float(*)[SB::kFloats]>(lds + 2 * SA::kFloats);

    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;
    const int ntiles = p.tiles_m * p.tiles_n;
    const int total = ntiles * p.batch;
    const int step = gridDim.x;
    int w = blockIdx.x;
    if (w >= total) return;  // the host launches at most `total` workgroups

    const int ktiles = (p.k + BK - 1) / BK;  // >= 1: the host sends K = 0 to the plain kernels
    const int lda = (int)p.lda, ldb = (int)p.ldb;
    constexpr int RA = WA == 16 ? 3 : 0, RB = WB == 16 ? 3 : 0;
    const uint32_t a_bytes = (uint32_t)(AK ? (p.m - 1) * lda + ((p.k + RA) & ~RA) : (p.k - 1) * lda + ((p.m + RA) & ~RA)) * 4u;
    const uint32_t b_bytes = (uint32_t)(BKC ? (p.n - 1) * ldb + ((p.k + RB) & ~RB) : (p.k - 1) * ldb + ((p.n + RB) & ~RB)) * 4u;

    // work item -> problem and tile origin (wave-uniform)
    auto decode = [&](int wi, int &bz, int &m0, int &n0) {
        bz = wi / ntiles;
        const int pid = wi - bz * ntiles;
        const int tm = pid / p.tiles_n;
        m0 = tm * BM;
        n0 = (pid - tm * p.tiles_n) * BN;
    };
    auto issue = [&](int bz, int m0, int n0, int k0, int st) {
        SA::issue(make_rsrc(p.a + (int64_t)bz * p.stride_a, a_bytes), lds_a[st], lda, m0, k0, p.m, p.k, wave, lane);
        SB::issue(make_rsrc(p.b + (int64_t)bz * p.stride_b, b_bytes), lds_b[st], ldb, n0, k0, p.n, p.k, wave, lane);
    };

    zn_f32x16 acc[FM][FN];
    {
        int bz, m0, n0;
        decode(w, bz, m0, n0);
        issue(bz, m0, n0, 0, 0);
    }
    int stage = 0;
    bool after_interior = false;  // the previous tile's epilogue issued >= S stores after the prefetch
    for (;;) {
        int bz, m0, n0;
        decode(w, bz, m0, n0);
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0.0f;
        const bool has_next = w + step < total;
        for (int kt = 0; kt < ktiles; ++kt) {
            if (kt == 0 && after_interior)
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(S) : "memory");  // the prefetch has landed
            else
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();  // every wave's part of this stage is in LDS; the other stage is free
            if (kt + 1 < ktiles) {
                issue(bz, m0, n0, (kt + 1) * BK, stage ^ 1);
            } else if (has_next) {  // the next tile's first slice
                int bz2, m2, n2;
                decode(w + step, bz2, m2, n2);
                issue(bz2, m2, n2, 0, stage ^ 1);
            }
            const float *la = lds_a[stage];
            const float *lb = lds_b[stage];
#pragma unroll
            for (int kg = 0; kg < BK; kg += 8) {
                float fa[FM][4], fb[FN][4];
                read_frags_dma<BM, BK, FM, AK>(la, wm0, kg, lane, fa);
                read_frags_dma<BN, BK, FN, BKC>(lb, wn0, kg, lane, fb);
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                        for (int fn = 0; fn < FN; ++fn)
                            acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[fm][t], fb[fn][t], acc[fm][fn], 0, 0, 0);
            }
            stage ^= 1;
        }
        store_tile_act<BM, BN, WM, WN, AK, BKC, ACT, true>(p, acc, bz, m0, n0, wm0, wn0, lane, 0);
        if (!has_next) break;
        after_interior = m0 + BM <= p.m && n0 + BN <= p.n;
        w += step;
    }
}

// The persistent GEMM with deferred stores, for plain problems (no bias,
// no accumulation, linear) whose tiles all lie inside C and span at least
// kSpread = 4 K slices: a finished tile's results move to a second set of
// registers and are stored during the first four slices of the workgroup's
// next tile, an eighth after each of their k groups, instead of in one
// burst at the end of the tile (C5's QK^T, K = 64: the bursts stalled the
// next tiles' loads).  Each slice wait leaves the previous slice's stores in
// flight: the only operations issued after a slice's DMA are those stores,
// a fixed number (kPerSlice) for an interior tile.  The workgroup's last
// tile is stored directly.  Each element sums K in the same order as
// gemm_persistent, so the results are the same bits.  KT > 0: K is exactly
// KT slices (the host checks), so the slice loop unrolls and every store
// group and wait is fixed at compile time.
template <int BM, int BN, int BK, int WM, int WN, bool AK, bool BKC, int KT = 0>
__device__ __forceinline__ void gemm_persistent_defer(const ZnGemmArgs &p, float *lds) {
    constexpr int NT = WM * WN * kWave;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    // A K-contiguous B is read X-permuted (lane j: columns FN j .. FN j + FN - 1),
    // so that every layout stores FN consecutive columns per lane
    constexpr bool kXP = BKC && FN > 1;
    constexpr bool kVec = FN > 1;
    constexpr int kItems = FM * 16;                 // (fm, r) row items of a wave tile
    constexpr int kSpread = 4;                      // slices the stores of a tile are spread over
    constexpr int kGroup = kItems / (2 * kSpread);  // items stored after each k group
    constexpr int kPerSlice = 2 * kGroup * (kVec ? 1 : FN);  // store instructions issued in one slice
    static_assert(kItems % (2 * kSpread) == 0 && kPerSlice < 64, "equal store groups within the vmcnt range");
    static_assert(BK == 16, "two k groups per slice, one store group after each");
    typedef DmaStage<BM, BK, NT, AK, 16> SA;
    typedef DmaStage<BN, BK, NT, BKC, 16> SB;
    float(*lds_a)[SA::kFloats] = reinterpret_cast<float(*)[SA::kFloats]>(lds);
    float(*lds_b)[SB::kFloats] = reinterpret_cast<float(*)[SB::kFloats]>(lds + 2 * SA::kFloats);

    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;
    const int j = lane & 31, h = lane >> 5;
    const int ntiles = p.tiles_m * p.tiles_n;
    const int total = ntiles * p.batch;
    // Work items walked by this workgroup: w, w + step, ... below `end`.
    // xcd_remap 3 (at least 8 workgroups): the items are cut into 8 equal
    // contiguous chunks and XCD x's workgroups (linear ids x, x + 8, ...,
    // dispatched to XCD x) walk chunk x, so the tiles running at once on one
    // XCD belong to the same few problems and share their operand panels in
    // that XCD's L2.  Either walk covers every item once.
    int w = blockIdx.x, step = gridDim.x, end = total;
    if (p.xcd_remap == 3) {
        const int x = (int)blockIdx.x & 7;
        const int begin = (int)((int64_t)total * x / 8);
        end = (int)((int64_t)total * (x + 1) / 8);
        step = ((int)gridDim.x - x + 7) / 8;  // workgroups on XCD x
        w = begin + ((int)blockIdx.x >> 3);
    }
    if (w >= end) return;  // the host launches at most `total` workgroups

    const int ktiles = KT > 0 ? KT : (p.k + BK - 1) / BK;  // >= kSpread: the host sends shorter K to gemm_persistent
    const int lda = (int)p.lda, ldb = (int)p.ldb;
    const uint32_t a_bytes = (uint32_t)(AK ? (p.m - 1) * lda + ((p.k + 3) & ~3) : (p.k - 1) * lda + ((p.m + 3) & ~3)) * 4u;
    const uint32_t b_bytes = (uint32_t)(BKC ? (p.n - 1) * ldb + ((p.k + 3) & ~3) : (p.k - 1) * ldb + ((p.n + 3) & ~3)) * 4u;

    auto decode = [&](int wi, int &bz, int &m0, int &n0) {
        bz = wi / ntiles;
        const int pid = wi - bz * ntiles;
        const int tm = pid / p.tiles_n;
        m0 = tm * BM;
        n0 = (pid - tm * p.tiles_n) * BN;
    };
    // The lane's DMA byte offsets at k = 0 of a tile are computed once per
    // tile (masked on M and N); slice s adds s times an increment, and K is
    // masked only in a partial last slice (an out-of-range offset plus
    // s * inc stays past the operand, which is below 2^31 bytes).
    constexpr int LA = SA::kPerWave, LB = SB::kPerWave;
    const uint32_t inca = (uint32_t)(AK ? BK : BK * lda) * 4u, incb = (uint32_t)(BKC ? BK : BK * ldb) * 4u;
    auto chunk = [&](int q, int kwaves, int per_inst) { return (q * kwaves + wave) * per_inst + 4 * lane; };
    auto tile_offsets = [&](int m0, int n0, uint32_t(&oa)[LA], uint32_t(&ob)[LB]) {
#pragma unroll
        for (int q = 0; q < LA; ++q) {
            const int c = chunk(q, SA::kWaves, SA::kPerInst);
            const int outer = AK ? m0 + c / BK : c / BM;
            const int inner = AK ? 4 * (((c % BK) / 4) ^ SA::swz(c / BK)) : m0 + c % BM;
            oa[q] = (AK ? outer < p.m : inner < p.m) ? (uint32_t)(outer * lda + inner) * 4u : kOutOfRange;
        }
#pragma unroll
        for (int q = 0; q < LB; ++q) {
            const int c = chunk(q, SB::kWaves, SB::kPerInst);
            const int outer = BKC ? n0 + c / BK : c / BN;
            const int inner = BKC ? 4 * (((c % BK) / 4) ^ SB::swz(c / BK)) : n0 + c % BN;
            ob[q] = (BKC ? outer < p.n : inner < p.n) ? (uint32_t)(outer * ldb + inner) * 4u : kOutOfRange;
        }
    };
    const uint32_t lds_a0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(zn_lds_void *)&lds_a[0][0]);
    const uint32_t lds_b0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(zn_lds_void *)&lds_b[0][0]);
    auto issue = [&](int bz, const uint32_t(&oa)[LA], const uint32_t(&ob)[LB], int s, int st) {
        const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + (int64_t)bz * p.stride_a, a_bytes);
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b + (int64_t)bz * p.stride_b, b_bytes);
        const int k0 = s * BK;
        const bool partial = k0 + BK > p.k;
#pragma unroll
        for (int q = 0; q < LA; ++q) {
            uint32_t off = oa[q] + (uint32_t)s * inca;
            if (partial) {
                const int c = chunk(q, SA::kWaves, SA::kPerInst);
                const int kk = AK ? k0 + 4 * (((c % BK) / 4) ^ SA::swz(c / BK)) : k0 + c / BM;
                if (kk >= p.k) off = kOutOfRange;
            }
            const uint32_t dst = lds_a0 + (uint32_t)(st * SA::kFloats + (q * SA::kWaves + wave) * SA::kPerInst) * 4u;
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" : : "s"(dst), "v"(off), "s"(ra) : "memory");
        }
#pragma unroll
        for (int q = 0; q < LB; ++q) {
            uint32_t off = ob[q] + (uint32_t)s * incb;
            if (partial) {
                const int c = chunk(q, SB::kWaves, SB::kPerInst);
                const int kk = BKC ? k0 + 4 * (((c % BK) / 4) ^ SB::swz(c / BK)) : k0 + c / BN;
                if (kk >= p.k) off = kOutOfRange;
            }
            const uint32_t dst = lds_b0 + (uint32_t)(st * SB::kFloats + (q * SB::kWaves + wave) * SB::kPerInst) * 4u;
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" : : "s"(dst), "v"(off), "s"(rb) : "memory");
        }
    };
    // Non-temporal stores of row items [i0, i1) of v, a tile at (bz, m0, n0):
    // buffer stores into one problem's C (below 2^31 bytes), the lane's byte
    // offset at the wave tile's first row in a vector register and each
    // item's row offset in a scalar one, so an item costs its store alone.
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    constexpr int kNt = 2;  // the nt cache-policy bit of the raw buffer builtins
    const uint32_t ldc4 = (uint32_t)p.ldc * 4u;
    const uint32_t c_bytes = (uint32_t)((p.m - 1) * p.ldc + p.n) * 4u;
    auto store_items = [&](const zn_f32x16(&v)[FM][FN], int bz, int m0, int n0, int i0, int i1) {
        float *gc = p.c + (int64_t)bz * p.stride_c;
        if constexpr (kVec && FN == 4) {
            const __amdgpu_buffer_rsrc_t rc = make_rsrc(gc, c_bytes);
            const uint32_t voff =
                ((uint32_t)(m0 + wm0 + (AK ? 4 * h : FM * 4 * h)) * (uint32_t)p.ldc + (uint32_t)(n0 + wn0 + FN * j)) * 4u;
#pragma unroll
            for (int it = 0; it < kItems; ++it) {
                if (it < i0 || it >= i1) continue;
                const int fm = it >> 4, r = it & 15;
                const int rr = 8 * (r >> 2) + (r & 3);
                const int irow = AK ? 32 * fm + rr : FM * rr + fm;
                const zn_f32x4 x = {v[fm][0][r], v[fm][1][r], v[fm][2][r], v[fm][3][r]};
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), rc, voff, (uint32_t)irow * ldc4, kNt);
            }
            return;
        }
#pragma unroll
        for (int it = 0; it < kItems; ++it) {
            if (it < i0 || it >= i1) continue;
            const int fm = it >> 4, r = it & 15;
            const int bi = 8 * (r >> 2) + 4 * h + (r & 3);
            const int row = m0 + wm0 + (AK ? 32 * fm + bi : FM * bi + fm);
            float *crow = gc + (int64_t)row * p.ldc;
            if constexpr (kVec) {
                typedef typename FVec<FN>::type VT;
                VT x;
#pragma unroll
                for (int fn = 0; fn < FN; ++fn) x[fn] = v[fm][fn][r];
                __builtin_nontemporal_store(x, reinterpret_cast<VT *>(crow + n0 + wn0 + FN * j));
            } else {
#pragma unroll
                for (int fn = 0; fn < FN; ++fn)
                    __builtin_nontemporal_store(v[fm][fn][r], crow + n0 + wn0 + (BKC ? 32 * fn + j : FN * j + fn));
            }
        }
    };

    zn_f32x16 acc[FM][FN], pend[FM][FN];
    int pbz = 0, pm0 = 0, pn0 = 0;
    bool pending = false;      // pend holds a tile to store during this tile's first kSpread slices
    bool stored_last = false;  // the previous slice issued stores after this slice's DMA
    int bz, m0, n0;            // the current tile, and its DMA offsets
    uint32_t ca[LA], cb[LB];
    decode(w, bz, m0, n0);
    tile_offsets(m0, n0, ca, cb);
    issue(bz, ca, cb, 0, 0);
    int stage = 0;
    for (;;) {
        int nbz = 0, nm0 = 0, nn0 = 0;  // the next tile, and its DMA offsets
        uint32_t na[LA], nb[LB];
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0.0f;
        const bool has_next = w + step < end;
#pragma unroll
        for (int kt = 0; kt < ktiles; ++kt) {
            if (stored_last)
                vm_wait<kPerSlice>();  // slice kt has landed; the previous slice's stores may still be in flight
            else
                vm_wait<0>();
            stored_last = pending && kt < kSpread;
            __syncthreads();  // every wave's part of this stage is in LDS; the other stage is free
            if (kt + 1 < ktiles) {
                issue(bz, ca, cb, kt + 1, stage ^ 1);
            } else if (has_next) {  // the next tile's first slice
                decode(w + step, nbz, nm0, nn0);
                tile_offsets(nm0, nn0, na, nb);
                issue(nbz, na, nb, 0, stage ^ 1);
            }
            const float *la = lds_a[stage];
            const float *lb = lds_b[stage];
#pragma unroll
            for (int kg = 0; kg < BK; kg += 8) {
                float fa[FM][4], fb[FN][4];
                read_frags_dma<BM, BK, FM, AK>(la, wm0, kg, lane, fa);
                read_frags_dma<BN, BK, FN, BKC, kXP>(lb, wn0, kg, lane, fb);
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                        for (int fn = 0; fn < FN; ++fn)
                            acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[fm][t], fb[fn][t], acc[fm][fn], 0, 0, 0);
                if (pending && kt < kSpread) {  // an eighth of the previous tile after each k group
                    const int q = kt * 2 + kg / 8;
                    store_items(pend, pbz, pm0, pn0, q * kGroup, (q + 1) * kGroup);
                }
            }
            stage ^= 1;
        }
        if (!has_next) {
            store_items(acc, bz, m0, n0, 0, kItems);
            break;
        }
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) pend[fm][fn] = acc[fm][fn];
        pbz = bz;
        pm0 = m0;
        pn0 = n0;
        pending = true;
        w += step;
        bz = nbz;
        m0 = nm0;
        n0 = nn0;
#pragma unroll
        for (int q = 0; q < LA; ++q) ca[q] = na[q];
#pragma unroll
        for (int q = 0; q < LB; ++q) cb[q] = nb[q];
    }
}

}  // namespace

#endif  // ZN_GEMM_CORE_H
