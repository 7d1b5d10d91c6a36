// Shared device helpers of the MFMA kernels (GEMM, convolution, attention):
// vector types, raw buffer descriptors, X-contiguous fragment reads and the
// LDS-DMA operand staging.  Included by each kernel translation unit; every
// definition has internal linkage.
#ifndef ZN_MFMA_STAGE_H
#define ZN_MFMA_STAGE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef float zn_f32x16 __attribute__((ext_vector_type(16)));
typedef float zn_f32x4 __attribute__((ext_vector_type(4)));
typedef float zn_f32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

template <int N> struct FVec;
template <> struct FVec<1> { typedef float type; };
template <> struct FVec<2> { typedef zn_f32x2 type; };
template <> struct FVec<4> { typedef zn_f32x4 type; };

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
    static_assert(!KC || BK == 16 || BK == 32 || BK == 64 || BK == 128, "K-contiguous DMA staging: BK 16..128");

    // K-contiguous operands are stored [x][BK] without padding; chunk c (4
    // floats) of row x sits in slot c ^ swz(x), so that 16 consecutive rows
    // (one 16-lane group of a fragment read) land in 16 distinct 16-byte
    // groups of a 256-byte bank span (rows are BK*4 bytes, so 64/BK of them
    // share a span; swz spreads those over its chunks).  Spreading only 8
    // rows left 2-way conflicts: SQ_LDS_BANK_CONFLICT of the 8192^3 GEMM went
    // from 1.3e8 cycles to 0 with this layout.  X-contiguous operands are
    // stored [BK][BX].
    __device__ static __forceinline__ int swz(int row) {
        if constexpr (BK == 16) return (row >> 2) & 3;  // 4 rows per 256 bytes, 4 chunks per row
        else if constexpr (BK == 32) return (row >> 1) & 7;  // 2 rows per 256 bytes, 8 chunks per row
        else return row & 15;  // one row spans 256 bytes or more
    }

    // Instruction j of a wave covers outer indices kStep further than
    // instruction j - 1 (its inner index, which the swizzle may change, is
    // computed as before), so outer * ld is the first instruction's plus
    // j * kStep * ld: one multiply per stage, not per load.
    static constexpr int kStep = KC ? kWaves * kPerInst / BK : kWaves * kPerInst / BX;
    static constexpr bool kStrided = (KC ? (kWaves * kPerInst) % BK : (kWaves * kPerInst) % BX) == 0;

    __device__ static __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, float *lds, int ld, int x0, int k0,
                                                 int xmax, int kmax, int wave, int lane) {
        const int step_ld = kStep * ld;
        int outer_ld0 = 0;  // outer * ld of instruction 0
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
            int lin;
            if constexpr (kStrided) {
                if (j == 0) outer_ld0 = outer * ld;
                lin = outer_ld0 + j * step_ld + inner;
            } else {
                lin = outer * ld + inner;
            }
            const uint32_t off = ok ? (uint32_t)lin * 4u : kOutOfRange;
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


// Fragments from the staged LDS tile: a K-contiguous tile gives one 16-byte
// read per block (lane i: row w0 + 32f + i, k = kg + 4h .. kg + 4h + 3).
// XP: lane i of block f takes row w0 + FX * i + f instead, so that a lane
// holds FX consecutive rows (of B: consecutive columns of C).
template <int BX, int BK, int FX, bool KC, bool XP = false>
__device__ __forceinline__ void read_frags_dma(const float *lds, int w0, int kg, int lane, float (&frag)[FX][4]) {
    if constexpr (KC) {
        const int i = lane & 31;
        const int h = lane >> 5;
#pragma unroll
        for (int f = 0; f < FX; ++f) {
            const int row = XP ? w0 + FX * i + f : w0 + 32 * f + i;
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

// One LDS read of the fragments read_frags_dma reads for a K group: for a
// K-contiguous tile, block `idx` (one 16-byte read of 4 consecutive k); for an
// X-contiguous tile, MFMA step `idx` (one FX-wide read of FX consecutive rows).
// Lets a main loop spread a group's reads over the MFMAs of the previous one.
template <int BX, int BK, int FX, bool KC>
__device__ __forceinline__ void read_frag_one(const float *lds, int w0, int kg, int lane, int idx, float (&frag)[FX][4]) {
    const int i = lane & 31;
    const int h = lane >> 5;
    if constexpr (KC) {
        const int row = w0 + 32 * idx + i;
        const int slot = (kg / 4 + h) ^ DmaStage<BX, BK, kWave, true, 16>::swz(row);
        const zn_f32x4 v = *reinterpret_cast<const zn_f32x4 *>(lds + row * BK + 4 * slot);
        frag[idx][0] = v[0];
        frag[idx][1] = v[1];
        frag[idx][2] = v[2];
        frag[idx][3] = v[3];
    } else {
        typedef typename FVec<FX>::type VT;
        const VT v = *reinterpret_cast<const VT *>(lds + (kg + 4 * h + idx) * BX + w0 + FX * i);
        if constexpr (FX == 1) {
            frag[0][idx] = v;
        } else {
#pragma unroll
            for (int f = 0; f < FX; ++f) frag[f][idx] = v[f];
        }
    }
}

}  // namespace

#endif
