// fp32 GEMM for gfx950 (CDNA4) on the fp32 matrix cores.
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
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../zn_kernel_args.h"

typedef float zn_f32x16 __attribute__((ext_vector_type(16)));
typedef float zn_f32x4 __attribute__((ext_vector_type(4)));
typedef float zn_f32x2 __attribute__((ext_vector_type(2)));

namespace {

constexpr int kWave = 64;

template <int N> struct FVec;
template <> struct FVec<1> { typedef float type; };
template <> struct FVec<2> { typedef zn_f32x2 type; };
template <> struct FVec<4> { typedef zn_f32x4 type; };

__device__ __forceinline__ float zn_activate(float v, int act) {
    switch (act) {
    case 1: return v > 0.0f ? v : 0.0f;               // relu   (src/backend.zig:239-240)
    case 2: return 1.0f / (1.0f + expf(-v));          // sigmoid (src/backend.zig:264-265)
    case 3: return tanhf(v);                          // tanh   (src/backend.zig:289-290)
    default: return v;
    }
}

// Raw buffer descriptor over one operand of one problem: loads at byte
// offsets >= `bytes` return zero, so masked elements use an out-of-range
// offset instead of a branch.
constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const float *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, (int)bytes, 0x00020000);
}

// Fragments for the four MFMA steps of one K group of 8 from an
// X-contiguous LDS tile [BK][BX]: frag[f][t] is the operand value of lane
// (i = lane % 32, h = lane / 32) for block f at k = kg + 4h + t; lane i owns
// rows w0 + FX*i + f, f < FX, so each step is one FX-wide LDS read.
template <int BX, int BK, int FX>
__device__ __forceinline__ void read_frags_x(const float *lds, int w0, int kg, int lane, float (&frag)[FX][4]) {
    const int i = lane & 31;
    const int h = lane >> 5;
    typedef typename FVec<FX>::type VT;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const VT v = *reinterpret_cast<const VT *>(lds + (kg + 4 * h + t) * BX + w0 + FX * i);
        if constexpr (FX == 1) {
            frag[0][t] = v;
        } else {
#pragma unroll
            for (int f = 0; f < FX; ++f) frag[f][t] = v[f];
        }
    }
}

// ---- operand staging straight into LDS -----------------------------------
// buffer_load_dwordx4 ... lds writes lane L's 16 bytes to LDS address
// M0 + 16*L (buffer_load_dword ... lds: 4 bytes at M0 + 4*L), so one wave
// instruction fills a contiguous 1 KB (256 B) block; lanes with an
// out-of-range offset write zeros (both behaviours checked on gfx950).  The loads are issued from inline assembly so that the compiler
// does not guard every LDS read with a wait for all outstanding loads; the
// kernel waits explicitly (vmcnt) before each stage's barrier.  M0 is set
// immediately before each load and is not used by any other code in these
// kernels (the build emits the assembly and tests/test_abi.py checks it).
typedef __attribute__((address_space(3))) void zn_lds_void;

template <int BX, int BK, int NT, bool KC, int W>
struct DmaStage {
    static_assert(W == 16 || W == 4, "16-byte or 4-byte loads");
    static constexpr int kFloats = BX * BK;
    static constexpr int kPerInst = W / 4 * kWave;  // floats one wave instruction writes (256 or 64)
    static constexpr int kInsts = kFloats / kPerInst;
    static constexpr int kWaves = NT / kWave;
    static constexpr int kPerWave = kInsts / kWaves;
    static_assert(kInsts % kWaves == 0 && kPerWave >= 1, "load blocks must split evenly over waves");
    static_assert(!KC || BK == 16 || BK == 32, "K-contiguous DMA staging supports BK 16 and 32");

    // K-contiguous operands are stored [x][BK] without padding; chunk c (4
    // floats) of row x sits in slot c ^ swz(x), which spreads the 16-byte
    // fragment reads of 8 consecutive rows over all banks.  X-contiguous
    // operands are stored [BK][BX].
    __device__ static __forceinline__ int swz(int row) { return BK == 16 ? ((row >> 1) & 3) : (row & 7); }

    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, float *lds, int ld, int x0, int k0,
                                                 int xmax, int kmax, int wave, int lane) {
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int p0 = (j * kWaves + wave) * kPerInst;  // first LDS float this instruction writes
            int outer, inner;
            bool ok;
            if constexpr (W == 16) {
                const int p = p0 + 4 * lane;  // lane writes LDS floats p .. p + 3
                if constexpr (KC) {
                    const int row = p / BK;
                    const int c = ((p % BK) / 4) ^ swz(row);
                    outer = x0 + row;
                    inner = k0 + 4 * c;
                } else {
                    outer = k0 + p / BX;
                    inner = x0 + p % BX;
                }
                ok = outer < (KC ? xmax : kmax) && inner < (KC ? kmax : xmax);
            } else {
                const int p = p0 + lane;  // lane writes LDS float p
                if constexpr (KC) {
                    const int row = p / BK, pos = p % BK;
                    const int c = (pos / 4) ^ swz(row);
                    outer = x0 + row;
                    inner = k0 + 4 * c + (pos & 3);
                } else {
                    outer = k0 + p / BX;
                    inner = x0 + p % BX;
                }
                ok = outer < (KC ? xmax : kmax) && inner < (KC ? kmax : xmax);
            }
            const uint32_t off = ok ? (uint32_t)(outer * ld + inner) * 4u : kOutOfRange;
            const uint32_t lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(zn_lds_void *)(lds + p0));
            if constexpr (W == 16)
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                             :
                             : "s"(lds_addr), "v"(off), "s"(rsrc)
                             : "memory");
            else
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                             :
                             : "s"(lds_addr), "v"(off), "s"(rsrc)
                             : "memory");
        }
    }
};

// Implicit-GEMM convolution operand: the X-contiguous tile [BK][BN] of the
// virtual im2col matrix, element (k, n) gathered with 4-byte loads from the
// NCHW input (out-of-image taps and out-of-problem elements read zero).  One
// wave instruction covers 64 consecutive n of one k row when BN >= 64, so
// the filter-tap decode is uniform across the wave.
template <int BN, int BK, int NT>
struct ConvGatherStage {
    static constexpr int kFloats = BN * BK;
    static constexpr int kInsts = kFloats / kWave;
    static constexpr int kWaves = NT / kWave;
    static constexpr int kPerWave = kInsts / kWaves;
    static_assert(kInsts % kWaves == 0 && kPerWave >= 1, "load blocks must split evenly over waves");

    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, float *lds, const ZnConvGeom &g,
                                                 int n0, int k0, int nmax, int kmax, int wave, int lane) {
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int p0 = (j * kWaves + wave) * kWave;
            const int pos = p0 + lane;
            const int k = k0 + pos / BN;
            const int n = n0 + pos % BN;
            int ic, kh, kw;
            if (g.k_order == 0) {
                const int kpos = k / g.channels;
                ic = k - kpos * g.channels;
                kh = kpos / g.k_w;
                kw = kpos - kh * g.k_w;
            } else {
                const int khw = g.k_h * g.k_w;
                ic = k / khw;
                const int kpos = k - ic * khw;
                kh = kpos / g.k_w;
                kw = kpos - kh * g.k_w;
            }
            const int oh = n / g.out_w, ow = n - oh * g.out_w;
            const int ih = oh * g.stride_h - g.pad_h + kh;
            const int iw = ow * g.stride_w - g.pad_w + kw;
            const bool ok = n < nmax && k < kmax && (unsigned)ih < (unsigned)g.in_h && (unsigned)iw < (unsigned)g.in_w;
            const uint32_t off = ok ? (uint32_t)((ic * g.in_h + ih) * g.in_w + iw) * 4u : kOutOfRange;
            const uint32_t lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(zn_lds_void *)(lds + p0));
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                         :
                         : "s"(lds_addr), "v"(off), "s"(rsrc)
                         : "memory");
        }
    }
};

// Fragments from the staged LDS tile: a K-contiguous tile gives one 16-byte
// read per block (lane i: row w0 + 32f + i, k = kg + 4h .. kg + 4h + 3).
template <int BX, int BK, int FX, bool KC>
__device__ __forceinline__ void read_frags_dma(const float *lds, int w0, int kg, int lane, float (&frag)[FX][4]) {
    if constexpr (KC) {
        const int i = lane & 31;
        const int h = lane >> 5;
#pragma unroll
        for (int f = 0; f < FX; ++f) {
            const int row = w0 + 32 * f + i;
            const int slot = (kg / 4 + h) ^ DmaStage<BX, BK, kWave, true, 16>::swz(row);
            const zn_f32x4 v = *reinterpret_cast<const zn_f32x4 *>(lds + row * BK + 4 * slot);
            frag[f][0] = v[0];
            frag[f][1] = v[1];
            frag[f][2] = v[2];
            frag[f][3] = v[3];
        }
    } else {
        read_frags_x<BX, BK, FX>(lds, w0, kg, lane, frag);
    }
}

// Tile coordinates of this workgroup: optional XCD-contiguous remap, then
// groups of `group_m` tile rows (group_m = 1 is plain row-major order).
__device__ __forceinline__ void tile_coords(const ZnGemmArgs &p, int &tm, int &tn) {
    int pid = blockIdx.x;
    const int ntiles = p.tiles_m * p.tiles_n;
    if (p.xcd_remap) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
    const int group_span = p.group_m * p.tiles_n;
    const int first_m = (pid / group_span) * p.group_m;
    const int gsize = min(p.tiles_m - first_m, p.group_m);
    const int in_group = pid % group_span;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// Epilogue of one macro tile: v = acc (+ C) (+ bias) -> act -> store.
// 32x32 accumulator layout: register r of lane (j = lane % 32, h = lane / 32)
// holds block row 8*(r/4) + 4*h + r%4, block column j.  A split-K slice
// stores its raw partial sums to the workspace instead.
template <int BM, int BN, int WM, int WN, bool AK, bool BKC>
__device__ __forceinline__ void store_tile(const ZnGemmArgs &p, const zn_f32x16 (&acc)[BM / WM / 32][BN / WN / 32],
                                           int m0, int n0, int wm0, int wn0, int lane) {
    constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
    const int64_t bz = blockIdx.y;
    float *gc = p.c + bz * p.stride_c;
    const bool split = p.splits > 1;
    if (split) gc = p.ws + ((int64_t)bz * p.splits + blockIdx.z) * (int64_t)p.m * p.n;
    const int64_t ldc = split ? (int64_t)p.n : p.ldc;
    const bool accumulate = !split && p.accumulate;
    const int act = split ? 0 : p.act;
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
                    crow[col] = zn_activate(x, act);
                }
            }
        }
    }
}

// The GEMM main loop: two LDS stages filled by DMA (WA/WB = 16: 16-byte
// loads for aligned operands, 4: 4-byte loads otherwise; CONV gathers B from
// an NCHW image).  Iteration kt waits
// for its stage (vmcnt(0) + barrier), refills the other stage with slice
// kt + 1, then computes slice kt while that load is in flight.
template <int BM, int BN, int BK, int WM, int WN, bool AK, bool BKC, int WA, int WB, bool CONV>
__device__ __forceinline__ void gemm_tile_dma(const ZnGemmArgs &p) {
    constexpr int NT = WM * WN * kWave;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
    static_assert(!CONV || (!BKC && WB == 4), "the convolution operand is X-contiguous and gathered");
    typedef DmaStage<BM, BK, NT, AK, WA> SA;
    typedef DmaStage<BN, BK, NT, BKC, WB> SB;
    typedef ConvGatherStage<BN, BK, NT> SC;
    __shared__ __attribute__((aligned(1024))) float lds_a[2][SA::kFloats];
    __shared__ __attribute__((aligned(1024))) float lds_b[2][SB::kFloats];

    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;
    int tm, tn;
    tile_coords(p, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int64_t bz = blockIdx.y;
    const float *ga = p.a + bz * p.stride_a;
    const float *gb = p.b + bz * p.stride_b;

    zn_f32x16 acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0.0f;

    const int kbeg = (int)blockIdx.z * p.k_chunk;
    const int kend = min(p.k, kbeg + p.k_chunk);
    const int ktiles = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int lda = (int)p.lda, ldb = (int)p.ldb;
    const uint32_t a_bytes = (uint32_t)(AK ? (p.m - 1) * lda + p.k : (p.k - 1) * lda + p.m) * 4u;
    const uint32_t b_bytes =
        CONV ? (uint32_t)(p.conv.channels * p.conv.in_h * p.conv.in_w) * 4u
             : (uint32_t)(BKC ? (p.n - 1) * ldb + p.k : (p.k - 1) * ldb + p.n) * 4u;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(ga, a_bytes);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(gb, b_bytes);

    auto issue_b = [&](float *lds, int k0) {
        if constexpr (CONV)
            SC::issue(rb, lds, p.conv, n0, k0, p.n, kend, wave, lane);
        else
            SB::issue(rb, lds, ldb, n0, k0, p.n, kend, wave, lane);
    };
    if (ktiles > 0) {
        SA::issue(ra, lds_a[0], lda, m0, kbeg, p.m, kend, wave, lane);
        issue_b(lds_b[0], kbeg);
    }
    for (int kt = 0; kt < ktiles; ++kt) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's part of slice kt is in LDS
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
    store_tile<BM, BN, WM, WN, AK, BKC>(p, acc, m0, n0, wm0, wn0, lane);
}

}  // namespace

// Exported kernels: zn_sgemm_<layout>_<tile>[_v].  Layout letters follow
// the reference: nn = Backend.matMul, nt = matMulTransposeB, tn =
// matMulTransposeA.  Tiles (macro tile, waves x wave tile):
//   x = 256x128, 8 waves of 64x64   large problems (two workgroups per CU)
//   l = 128x128, 4 waves of 64x64
//   n = 128x64,  2 waves of 64x64   narrow N (attention P.V, N = 64)
//   m = 64x64,   4 waves of 32x32   mid-size problems (BK 32)
//   s = 32x32,   1 wave             small problems (BK 32)
// The _v variants stage operands with 16-byte loads straight into LDS
// (aligned rows, contiguous extents a multiple of 4); the plain ones with
// 4-byte loads straight into LDS.
#define ZN_GEMM_KERNEL(NAME, BM, BN, BK, WM, WN, AK, BKC, VEC, MINB)                            \
    extern "C" __global__ __launch_bounds__(WM *WN * 64, MINB) void NAME(ZnGemmArgs p) {        \
        gemm_tile_dma<BM, BN, BK, WM, WN, AK, BKC, (VEC) ? 16 : 4, (VEC) ? 16 : 4, false>(p);    \
    }

#define ZN_GEMM_LAYOUTS(TILE, BM, BN, BK, WM, WN, MINB, VEC, SUFFIX)                            \
    ZN_GEMM_KERNEL(zn_sgemm_nn_##TILE##SUFFIX, BM, BN, BK, WM, WN, true, false, VEC, MINB)      \
    ZN_GEMM_KERNEL(zn_sgemm_nt_##TILE##SUFFIX, BM, BN, BK, WM, WN, true, true, VEC, MINB)       \
    ZN_GEMM_KERNEL(zn_sgemm_tn_##TILE##SUFFIX, BM, BN, BK, WM, WN, false, false, VEC, MINB)

#define ZN_GEMM_TILE(TILE, BM, BN, BK, WM, WN, MINB)                                            \
    ZN_GEMM_LAYOUTS(TILE, BM, BN, BK, WM, WN, MINB, true, _v)                                   \
    ZN_GEMM_LAYOUTS(TILE, BM, BN, BK, WM, WN, MINB, false, )

ZN_GEMM_TILE(x, 256, 128, 16, 4, 2, 1)
ZN_GEMM_TILE(l, 128, 128, 16, 2, 2, 4)
ZN_GEMM_TILE(n, 128, 64, 16, 2, 1, 1)
ZN_GEMM_TILE(m, 64, 64, 32, 2, 2, 1)
ZN_GEMM_TILE(s, 32, 32, 32, 1, 1, 1)

// Implicit-GEMM convolution, per image b = blockIdx.y:
// out_b[OC][OH*OW] = W[OC][K] . im2col(input_b)^T (+ bias[oc]), an NN GEMM
// whose B operand is gathered from the NCHW input (ZnConvGeom).  _v: W rows
// are 16-byte aligned.
#define ZN_CONV_KERNEL(TILE, BM, BN, BK, WM, WN, MINB, WA, SUFFIX)                                \
    extern "C" __global__ __launch_bounds__(WM *WN * 64, MINB) void zn_conv_nn_##TILE##SUFFIX(ZnGemmArgs p) { \
        gemm_tile_dma<BM, BN, BK, WM, WN, true, false, WA, 4, true>(p);                          \
    }
#define ZN_CONV_TILE(TILE, BM, BN, BK, WM, WN, MINB)                                              \
    ZN_CONV_KERNEL(TILE, BM, BN, BK, WM, WN, MINB, 16, _v)                                       \
    ZN_CONV_KERNEL(TILE, BM, BN, BK, WM, WN, MINB, 4, )

ZN_CONV_TILE(x, 256, 128, 16, 4, 2, 1)
ZN_CONV_TILE(l, 128, 128, 16, 2, 2, 4)
ZN_CONV_TILE(n, 128, 64, 16, 2, 1, 1)
ZN_CONV_TILE(m, 64, 64, 32, 2, 2, 1)
ZN_CONV_TILE(s, 32, 32, 32, 1, 1, 1)

// Split-K finish: C = act((accumulate ? C : 0) + sum over slices s = 0..S-1
// of ws[s] + bias[col or row]).  Slices are summed in ascending order, so results do not
// depend on scheduling.  Grid-stride over batch * m * n (float4 along n when
// n, ldc and C allow it).
extern "C" __global__ __launch_bounds__(256) void zn_splitk_reduce(ZnReduceArgs p) {
    const int64_t mn = (int64_t)p.m * p.n;
    const int vw = p.vec ? 4 : 1;
    const int64_t per_problem = mn / vw;
    const int64_t total = per_problem * p.batch;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = t / per_problem;
        const int64_t e = (t - b * per_problem) * vw;  // element index within the problem
        const int64_t row = e / p.n, col = e - row * p.n;
        const float *src = p.ws + b * p.splits * mn + e;
        float *dst = p.c + b * p.stride_c + row * p.ldc + col;
        if (p.vec) {
            zn_f32x4 s = *reinterpret_cast<const zn_f32x4 *>(src);
            for (int z = 1; z < p.splits; ++z) s = s + *reinterpret_cast<const zn_f32x4 *>(src + z * mn);
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
            for (int z = 1; z < p.splits; ++z) s = s + src[z * mn];
            float x = p.accumulate ? dst[0] + s : s;
            if (p.bias) x = x + p.bias[p.bias_rows ? row : col];
            dst[0] = zn_activate(x, p.act);
        }
    }
}
