// Fused single-pass attention for gfx950 on the fp32 matrix cores:
// O = softmax(scale * Q K^T) V per problem (one head, [seq_len x d_k] row
// major), the contract of cpuAttentionForward (src/backend.zig:3197-3222),
// without writing the [seq_len x seq_len] scores to memory.
//
// Each wave owns 32 queries and walks the keys in blocks of BKV, keeping a
// running row maximum and row sum (the online softmax): for every block
//   S^T = K_blk . (c Q)^T        (v_mfma_f32_32x32x2f32, K-dim = head dim)
//   m'  = max(m, max_key S^T),  P^T = exp2(S^T - m'),  c = scale*log2(e)
//   O^T = O^T * exp2(m - m') + V_blk^T . P^T,   l = l * exp2(m - m') + sum P
// and at the end O = O^T^T / l.
//
// Computing the transposed products makes the data flow register-only:
//  * the S^T accumulator (lane j + 32h, register r: key 8(r/4) + 4h + r%4 of a
//    32-key block, query j) is, register for register, the B operand of the
//    V^T . P^T product under the K order used by every kernel here (lane half
//    h, step t of K group g covers k = 8g + 4h + t);
//  * every value of query j lives in lanes j and j + 32, so the softmax
//    needs one cross-half exchange per block (the block maximum) and the
//    O^T rescale is lane-local.
// Q stays in registers for the whole walk; K and V blocks go HBM -> LDS by
// DMA (buffer_load ... lds, two stages, the same staging as the GEMM), K
// stored key-major [BKV][DP], V stored [BKV][DP] and read with the
// X-contiguous fragment rule (head dim d = FD*i + f for lane i, block f).
// Head dims are zero-padded to DP; keys past seq_len get score -inf.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../zn_kernel_args.h"

#include "zn_mfma_stage.h"

namespace {

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// One key block of the walk: S^T = K_blk . Q^T, the online-softmax update of
// (m, l, O^T) and O^T += V_blk^T . P^T.  MASK: the block runs past seq_len
// (only the last one can), its missing keys get score -inf.
template <int DP, int BKV, bool MASK>
__device__ __forceinline__ void attention_block(const float *lk, const float *lv, const float (&qf)[DP / 8][4],
                                                zn_f32x16 (&o)[DP / 32], float &m, float &l, int kv0, int S,
                                                int lane) {
    constexpr int FD = DP / 32;   // 32-row blocks of O^T (head dim)
    constexpr int FS = BKV / 32;  // 32-row blocks of S^T (keys)
    const int h = lane >> 5;
    zn_f32x16 s[FS];
#pragma unroll
    for (int f = 0; f < FS; ++f)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[f][r] = 0.0f;
#pragma unroll
    for (int g = 0; g < DP / 8; ++g) {
        float kf[FS][4];
        read_frags_dma<BKV, DP, FS, true>(lk, 0, 8 * g, lane, kf);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int f = 0; f < FS; ++f) s[f] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[f][t], qf[g][t], s[f], 0, 0, 0);
    }

    // scores are already in the log2 domain (Q was scaled by scale*log2(e))
    float mb = -INFINITY;
#pragma unroll
    for (int f = 0; f < FS; ++f)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            if constexpr (MASK)
                if (kv0 + 32 * f + 8 * (r / 4) + 4 * h + (r % 4) >= S) s[f][r] = -INFINITY;
            mb = fmaxf(mb, s[f][r]);
        }
    mb = fmaxf(mb, __shfl_xor(mb, 32));
    const float mn = fmaxf(m, mb);  // finite: every block holds at least one key
    const float alpha = exp2_fast(m - mn);
    float rs = 0.0f;
#pragma unroll
    for (int f = 0; f < FS; ++f)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float e = exp2_fast(s[f][r] - mn);
            s[f][r] = e;
            rs += e;
        }
    l = l * alpha + rs;
    m = mn;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {  // some query's maximum moved
#pragma unroll
        for (int f = 0; f < FD; ++f)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[f][r] *= alpha;
    }

    // O^T += V_blk^T . P^T; P^T is the S^T accumulator, register 4g + t
#pragma unroll
    for (int fs = 0; fs < FS; ++fs)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float vf[FD][4];
            read_frags_x<DP, BKV, FD>(lv, 0, 32 * fs + 8 * g, lane, vf);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int f = 0; f < FD; ++f)
                    o[f] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[f][t], s[fs][4 * g + t], o[f], 0, 0, 0);
        }
}

// Grid: blockIdx.x = problem, blockIdx.y = block of NW*32 queries, so the
// query blocks of one problem share an XCD and its L2 copy of K and V.
template <int DP, int BKV, int NW, int W>
__device__ __forceinline__ void attention_tile(const ZnAttnArgs &p) {
    constexpr int NT = NW * kWave;
    constexpr int FD = DP / 32;
    static_assert(DP % 32 == 0 && BKV % 32 == 0, "whole 32x32 blocks");
    typedef DmaStage<BKV, DP, NT, true, W> SK;   // K block, [key][d]
    typedef DmaStage<DP, BKV, NT, false, W> SV;  // V block, [key][d]
    __shared__ __attribute__((aligned(1024))) float lds_k[2][SK::kFloats];
    __shared__ __attribute__((aligned(1024))) float lds_v[2][SV::kFloats];

    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int j = lane & 31, h = lane >> 5;
    const int S = p.seq_len, D = p.d_k;
    const int64_t base = (int64_t)blockIdx.x * p.stride;
    const float *gq = p.q + base;
    const int q = (int)blockIdx.y * (NW * 32) + wave * 32 + j;  // this lane's query

    // Q^T fragments, the B operand of S^T = K . Q^T: qf[g][t] = Q[q][8g + 4h + t] * scale*log2(e).
    float qf[DP / 8][4];
#pragma unroll
    for (int g = 0; g < DP / 8; ++g) {
        const int f0 = 8 * g + 4 * h;
        if constexpr (W == 16) {
            zn_f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (q < S && f0 < D) v = *reinterpret_cast<const zn_f32x4 *>(gq + (int64_t)q * D + f0);
#pragma unroll
            for (int t = 0; t < 4; ++t) qf[g][t] = v[t] * p.scale_log2;
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t)
                qf[g][t] = (q < S && f0 + t < D) ? gq[(int64_t)q * D + f0 + t] * p.scale_log2 : 0.0f;
        }
    }

    zn_f32x16 o[FD];
#pragma unroll
    for (int f = 0; f < FD; ++f)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[f][r] = 0.0f;
    float m = -INFINITY;  // running maximum of this query's scaled scores (log2 domain)
    float l = 0.0f;       // this lane's share of the running sum

    const uint32_t bytes = (uint32_t)((int64_t)S * D * 4);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.k + base, bytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.v + base, bytes);
    const int nblk = (S + BKV - 1) / BKV;
    const int nfull = S / BKV;  // blocks with no missing keys
    SK::issue(rk, lds_k[0], D, 0, 0, S, D, wave, lane);
    SV::issue(rv, lds_v[0], D, 0, 0, D, S, wave, lane);
    for (int b = 0; b < nblk; ++b) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's part of block b is in LDS
        __syncthreads();  // every wave's part is; every wave is done with block b - 1
        const int cur = b & 1;
        if (b + 1 < nblk) {
            SK::issue(rk, lds_k[cur ^ 1], D, (b + 1) * BKV, 0, S, D, wave, lane);
            SV::issue(rv, lds_v[cur ^ 1], D, 0, (b + 1) * BKV, D, S, wave, lane);
        }
        if (b < nfull)
            attention_block<DP, BKV, false>(lds_k[cur], lds_v[cur], qf, o, m, l, b * BKV, S, lane);
        else
            attention_block<DP, BKV, true>(lds_k[cur], lds_v[cur], qf, o, m, l, b * BKV, S, lane);
    }

    // O[q][d] = O^T[d][q] / l.  Register r of block f holds d = FD*(8(r/4) + 4h + r%4) + f:
    // for each r/4 the lane owns the 4*FD consecutive head dims starting at FD*(8(r/4) + 4h).
    l += __shfl_xor(l, 32);
    if (q < S) {
        float *orow = p.out + base + (int64_t)q * D;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = FD * (8 * g + 4 * h);
            float vals[4 * FD];
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int f = 0; f < FD; ++f) vals[FD * t + f] = o[f][4 * g + t] / l;
            if constexpr (W == 16) {
#pragma unroll
                for (int c = 0; c < FD; ++c)
                    if (d0 + 4 * c < D)
                        *reinterpret_cast<zn_f32x4 *>(orow + d0 + 4 * c) =
                            zn_f32x4{vals[4 * c], vals[4 * c + 1], vals[4 * c + 2], vals[4 * c + 3]};
            } else {
#pragma unroll
                for (int e = 0; e < 4 * FD; ++e)
                    if (d0 + e < D) orow[d0 + e] = vals[e];
            }
        }
    }
}

}  // namespace

// zn_attention_d<DP>[_v]: head dims up to DP (zero-padded), 4 waves = 128
// queries per workgroup, blockIdx.x = problem, blockIdx.y = query block.  _v: 16-byte loads and stores
// (d_k % 4 == 0, 16-byte aligned Q, K, V and O).
#define ZN_ATTN_KERNEL(DP, BKV, W, SUFFIX)                                                   \
    extern "C" __global__ __launch_bounds__(256, 2) void zn_attention_d##DP##SUFFIX(ZnAttnArgs p) { \
        attention_tile<DP, BKV, 4, W>(p);                                                    \
    }
#define ZN_ATTN_DIM(DP, BKV)          \
    ZN_ATTN_KERNEL(DP, BKV, 16, _v)   \
    ZN_ATTN_KERNEL(DP, BKV, 4, )

ZN_ATTN_DIM(32, 64)
ZN_ATTN_DIM(64, 64)
ZN_ATTN_DIM(128, 32)
