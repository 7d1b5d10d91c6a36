// Two stacked Dense layers whose top layer is narrow (a classifier head of
// at most 16 outputs), fused across the layers: the forward of both layers
// in one launch and the backward of both in one launch.  The reference runs
// them layer by layer: Network.forward calls Dense.forward per layer
// (src/network.zig:309-360, src/layer.zig:380-409), and the backward loop
// calls Dense.backward per layer, top first (src/network.zig:455-477,
// src/layer.zig:411-475).  No workgroup ever waits for another.
//
// The kernels are latency-bound (a few us per launch), so the code avoids
// what serialises a wave: every load goes out before the first wait (raw
// buffer loads, out-of-range lanes read zero, no branches), and the work
// derived from the top layer (its K <= 16 products) runs on the matrix cores.
#include "gemm_core.h"

namespace {

__device__ __forceinline__ float bload(__amdgpu_buffer_rsrc_t r, bool ok, int elem) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, ok ? elem * 4 : (int)kOutOfRange, 0, 0));
}

__device__ __forceinline__ void bstore(__amdgpu_buffer_rsrc_t r, bool ok, int elem, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, ok ? elem * 4 : (int)kOutOfRange, 0, 0);
}

// activationBackward (src/optimization.zig:229-303) with the same expressions
// as zn_act_backward, so the same bits.  All four are computed and the
// activation's is kept by a bit-select whose masks (one all-ones, three
// zero) sit in vector registers the compiler cannot see into: with a
// visible activation id it turns the choice into branches, which split the
// batches of loads around them into one wait per element.  Zero inputs give
// +0 for every activation.
struct ActMask {
    uint32_t lin, relu, sig, th;
};

__device__ __forceinline__ uint32_t opaque_mask(bool on) {
    uint32_t v;
    asm("v_mov_b32 %0, %1" : "=v"(v) : "s"(on ? 0xffffffffu : 0u));
    return v;
}

__device__ __forceinline__ ActMask act_mask(int act) {
    return {opaque_mask(act == 0), opaque_mask(act == 1), opaque_mask(act == 2), opaque_mask(act == 3)};
}

__device__ __forceinline__ float act_backward_sel(float y, float go, const ActMask &m) {
    const float relu = y > 0.0f ? go : 0.0f;
    const float sig = (go * y) * (1.0f - y);
    const float th = go * (1.0f - y * y);
    return __builtin_bit_cast(float, (__builtin_bit_cast(uint32_t, go) & m.lin) |
                                         (__builtin_bit_cast(uint32_t, relu) & m.relu) |
                                         (__builtin_bit_cast(uint32_t, sig) & m.sig) |
                                         (__builtin_bit_cast(uint32_t, th) & m.th));
}

// Workgroup b of the grid runs on XCD b % 8 (the dispatcher deals them out
// in turn); with a grid of whole eights, the ids XCD x runs (x, x + 8, ...)
// are remapped to the contiguous range [x * G/8, (x + 1) * G/8), so that
// neighbouring tiles, which share operand blocks, share an L2.  Only the
// speed depends on this: the forward's 16 strips of C2 (two per XCD) took
// 6.99 -> 6.92 us; the backward's tiles lost with it (7.08 -> 7.37 us:
// its grad_x and grad_w1 tiles then crowd half the XCDs each).
__device__ __forceinline__ int xcd_contiguous(int b) {
    const int G = (int)gridDim.x;
    return (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
}

// ---------------------------------------------------------------- forward
// The forward's workgroup: eight waves (two per SIMD) split the lower
// layer's K over whole 32-slices as evenly as they go, each with one LDS
// stage (a slice is loaded, waited for and multiplied before the next is
// requested).  On MI355X, C2's forward (784-128-10, batch 256): four waves
// with every slice in flight 7.17 us; eight waves 6.44 us with four stages
// in flight, 6.48 with three, 6.33 with two, 6.18 with one; sixteen waves
// 6.40 (one stage) and 6.68 (two).  Requests in flight beyond the slice the
// wave needs next only delay that slice.
constexpr int kPairFwdWaves = 8;
constexpr int kPairFwdStages = 1;
// The lower layer runs on gemm_ksplit16's 16x16 tiles (the waves split K)
// and stores its block of h = act1(x . W1 + b1).  Each tile then multiplies
// that block by W2's 16 matching rows (one 16x16x4 MFMA step per 4 of K) into
// the tile's partial sum of the strip's y, writes the partial to the
// workspace as agent-scope atomic stores (coherent across the XCDs' L2
// caches), waits until they have completed, and arrives at its 16-row
// strip's counter.  The workgroup that arrives last, whichever it is, reads
// the strip's partials back with agent-scope loads (all in flight
// together), adds them in tile order, then the bias (after the whole sum,
// src/backend.zig:215) and the activation, and sets the counter back to zero,
// so nothing is cleared between launches and graph replays work.  Only the
// partials cross workgroups: h itself is written with ordinary stores.
template <int W, int ACT1>
__device__ __forceinline__ void pair_forward(const ZnPairFwdArgs &a, float *lds) {
    constexpr int KS = kPairFwdWaves;
    const ZnGemmArgs &p = a.l1;
    const int pid = xcd_contiguous((int)blockIdx.x);
    const int tm = pid / p.tiles_n, tn = pid - tm * p.tiles_n;
    const int m0 = tm * 16, n0 = tn * 16;
    const int t = threadIdx.x & 255, lane = threadIdx.x & 63;
    const bool elem = threadIdx.x < 256;  // threads 0..255 own one element of the 16x16 tile each
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int out = a.out;
    // 16x16x4 operands: in step s, lane (i, g = lane / 16) supplies A[i][4g + s]
    // (h) and B[4g + s][i] (W2's rows n0 ..); lane (j, g) receives row 4g + q,
    // column j of the product in register q.  W2 goes out before the main loop.
    const int i = lane & 15, g = lane >> 4;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w2, (uint32_t)(p.n * out) * 4u);
    float wv[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int k = n0 + 4 * g + s;
        wv[s] = bload(rw, wave == 0 && k < p.n && i < out, k * out + i);
    }
    // both biases go out before the main loop too, so that their latency hides
    const int row = m0 + (t >> 4), col = n0 + (t & 15);
    const float b1v = bload(make_rsrc(p.bias, p.bias ? (uint32_t)p.n * 4u : 0u), col < p.n, col);
    const float b2v = bload(make_rsrc(a.b2, a.b2 ? (uint32_t)out * 4u : 0u), (t & 15) < out, t & 15);
    float x = gemm_ksplit16_sum<KS, true, false, W, kPairFwdStages>(p, lds, m0, n0, 0);
    float hval = 0.0f;
    if (elem && row < p.m && col < p.n) {
        if (p.bias) x = x + b1v;
        hval = zn_activate(x, ACT1);
        p.c[(int64_t)row * p.ldc + col] = hval;
    }
    float *ht = lds + 4 * KS * 64;  // the h block, row stride 20 (gemm_ksplit16_sum's partials sit below)
    if (elem) ht[(t >> 4) * 20 + (t & 15)] = hval;
    __syncthreads();
    float *part = a.part + (int64_t)pid * 256;
    if (wave == 0) {
        const zn_f32x4 av = *reinterpret_cast<const zn_f32x4 *>(ht + i * 20 + 4 * g);
        zn_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s], wv[s], acc, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            __hip_atomic_store(part + (4 * g + q) * 16 + i, acc[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __shared__ int last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partial is written
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(a.counters + tm * kCounterStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               p.tiles_n - 1;
    __syncthreads();
    if (!last || !elem) return;
    if (t == 0) __hip_atomic_store(a.counters + tm * kCounterStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // thread t: y element (t / 16, t % 16) of the strip; the partials of the
    // strip's tiles, eight loads in flight at a time, added in tile order
    const float *strip = a.part + (int64_t)tm * p.tiles_n * 256 + t;
    float y = 0.0f;
    for (int t0 = 0; t0 < p.tiles_n; t0 += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            v[u] = __hip_atomic_load(strip + (int64_t)min(t0 + u, p.tiles_n - 1) * 256, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (t0 + u < p.tiles_n) y = t0 + u == 0 ? v[u] : y + v[u];
    }
    const int r = t >> 4, c = t & 15;
    if (m0 + r < p.m && c < out) {
        if (a.b2) y = y + b2v;
        a.y[(int64_t)(m0 + r) * out + c] = zn_activate(y, a.act2);
    }
}

// --------------------------------------------------------------- backward
// Every backward workgroup needs a few rows of W2 [hidden x out] and of
// grad_y (and y) [batch x out], out <= 16.  It copies the rows it needs
// into LDS once, all 256 threads together, 16 bytes at a time (the host
// takes this path only for 16-byte aligned W2, grad_y and y): "raw" copies,
// row-major, row stride out, zeros past the matrix, with gaa2 = act2'(y,
// grad_y) applied on the way in.  Every block of grad_h is read from them.
constexpr int kRawW = 2048, kRawG = 4096;  // floats of the W2 and gaa2 copies (checked on the host)

struct PairSrc {
    __amdgpu_buffer_rsrc_t h, w2, y, gy;
    int batch, hidden, out, act2;
    bool whole;  // hidden * out and batch * out are multiples of 4: no copy has a straddling float4
    ActMask m2;  // act2 for the bit-select of a non-linear head's derivative
};

__device__ __forceinline__ PairSrc pair_src(const ZnPairBwdArgs &a) {
    PairSrc s;
    s.h = make_rsrc(a.h, (uint32_t)(a.batch * a.hidden) * 4u);
    s.w2 = make_rsrc(a.w2, (uint32_t)(a.hidden * a.out) * 4u);
    s.y = make_rsrc(a.y, a.act2 ? (uint32_t)(a.batch * a.out) * 4u : 0u);  // read only for a non-linear head
    s.gy = make_rsrc(a.grad_y, (uint32_t)(a.batch * a.out) * 4u);
    s.batch = a.batch;
    s.hidden = a.hidden;
    s.out = a.out;
    s.act2 = a.act2;
    s.whole = ((a.hidden * a.out) & 3) == 0 && ((a.batch * a.out) & 3) == 0;
    s.m2 = act_mask(a.act2);
    return s;
}

__device__ __forceinline__ zn_f32x4 bload4(__amdgpu_buffer_rsrc_t r, bool ok, int elem) {
    return __builtin_bit_cast(zn_f32x4,
                              __builtin_amdgcn_raw_buffer_load_b128(r, ok ? elem * 4 : (int)kOutOfRange, 0, 0));
}

// One workgroup-wide copy: floats [base, base + len) of a matrix (base a
// multiple of 4), zero from `valid` on (relative to base); thread t takes
// floats 4 (t + 256u) .. + 3, u < 4 (len <= 4096), loading whole float4s
// that lie before `valid` and the one that straddles it float by float.
// Every copy's `valid` is a multiple of 4 when s.whole holds (the copies
// start at multiples of 32 rows and end at the matrix's end): then the
// straight-line path without the straddle runs.  Loaded into registers
// first (so that every load of the workgroup is in flight together), then
// written.
struct RawPart {
    zn_f32x4 v[4], y[4];
};

__device__ __forceinline__ zn_f32x4 raw_piece(__amdgpu_buffer_rsrc_t r, int base, int e, int valid) {
    zn_f32x4 v = bload4(r, e + 4 <= valid, base + e);
    if (e < valid && e + 4 > valid) {  // the one float4 that straddles the end of the matrix
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = bload(r, e + c < valid, base + e + c);
    }
    return v;
}

template <bool GAA>
__device__ __forceinline__ RawPart raw_load(const PairSrc &s, __amdgpu_buffer_rsrc_t r, int base, int len, int valid) {
    RawPart p;
    const int t = threadIdx.x;
    if (s.whole) {  // uniform
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = 4 * (t + 256 * u);
            const bool ok = e < len && e + 4 <= valid;
            p.v[u] = bload4(r, ok, base + e);
            if (GAA) p.y[u] = bload4(s.y, ok, base + e);
        }
        return p;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int e = 4 * (t + 256 * u);
        p.v[u] = raw_piece(r, base, e, e < len ? valid : 0);
        if (GAA) p.y[u] = raw_piece(s.y, base, e, e < len ? valid : 0);
    }
    return p;
}

template <bool GAA>
__device__ __forceinline__ void raw_store(const PairSrc &s, const RawPart &p, int len, float *raw) {
    const int t = threadIdx.x;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int e = 4 * (t + 256 * u);
        if (e < len) {
            zn_f32x4 v = p.v[u];
            if (GAA) {
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = act_backward_sel(p.y[u][c], v[c], s.m2);
            }
            *reinterpret_cast<zn_f32x4 *>(raw + e) = v;
        }
    }
}

// Block row of accumulator register q in lane half h (32x32x2 layout).
__device__ __forceinline__ int acc_row(int q, int h) { return 8 * (q >> 2) + 4 * h + (q & 3); }

// The 32x32 block of grad_h = gaa2 . W2^T for 32 batch rows (gaa2's raw
// rows g, row stride out) and 32 hidden columns (W2's raw rows w): the
// products over the head's k < out, two per v_mfma_f32_32x32x2f32 step
// (lane half h supplies k = 2s + h), in the same order in every workgroup,
// so every workgroup gets the same bits.  All LDS reads precede the MFMAs.
// Register q of lane (j, h) holds grad_h[batch row j][hidden column
// acc_row(q, h)].
__device__ __forceinline__ zn_f32x16 pair_grad_h(const float *w, const float *g, int out, int lane) {
    const int i = lane & 31, h = lane >> 5;
    const int steps = (out + 1) >> 1;  // uniform
    float xa[8], yb[8];
#pragma unroll
    for (int st = 0; st < 8; ++st) {
        const int k = 2 * st + h;
        const int kc = min(k, out - 1);  // stay inside the row; k >= out gives zero
        xa[st] = k < out ? w[i * out + kc] : 0.0f;
        yb[st] = k < out ? g[i * out + kc] : 0.0f;
    }
    zn_f32x16 d;
#pragma unroll
    for (int q = 0; q < 16; ++q) d[q] = 0.0f;
#pragma unroll
    for (int st = 0; st < 8; ++st)
        if (st < steps) d = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[st], yb[st], d, 0, 0, 0);
    return d;
}

// h in grad_h's register layout: lane (j, h) reads h[row][c0 + acc_row(q,
// h)] for q < 16, four groups of four consecutive columns.  WD 16: one
// 16-byte load per group (hidden a multiple of 4, aligned rows).
template <int WD>
__device__ __forceinline__ void h_load(const PairSrc &s, int row, int c0, int lane, float (&hv)[16]) {
    const int h = lane >> 5;
    if constexpr (WD == 16) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = c0 + 8 * e + 4 * h;
            const zn_f32x4 v = bload4(s.h, row < s.batch && c < s.hidden, row * s.hidden + c);
#pragma unroll
            for (int t = 0; t < 4; ++t) hv[4 * e + t] = v[t];
        }
    } else {
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int c = c0 + acc_row(q, h);
            hv[q] = bload(s.h, row < s.batch && c < s.hidden, row * s.hidden + c);
        }
    }
}

// gaa1 = act1'(h, grad_h) in grad_h's register layout.
template <int ACT1>
__device__ __forceinline__ void gaa1_of(const float (&hv)[16], const zn_f32x16 &d, float (&g)[16]) {
#pragma unroll
    for (int q = 0; q < 16; ++q) g[q] = zn_act_backward(hv[q], d[q], ACT1);
}

// A 32x32 block held in grad_h's register layout (lane j: block row j)
// written to LDS transposed, gt[column][row] (row stride kGt), and read back
// so that lane (n, h) gets gt[n][8e + 4h + t] in register 4e + t: the B
// fragments of a GEMM whose K runs over the block's rows, or column n's
// rows.  One wave, in order.
constexpr int kGt = 36;

__device__ __forceinline__ void transpose_block(const float (&g)[16], float *gt, int lane, float (&b)[16]) {
    const int j = lane & 31, h = lane >> 5;
#pragma unroll
    for (int q = 0; q < 16; ++q) gt[acc_row(q, h) * kGt + j] = g[q];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const zn_f32x4 v = *reinterpret_cast<const zn_f32x4 *>(gt + j * kGt + 8 * e + 4 * h);
#pragma unroll
        for (int t = 0; t < 4; ++t) b[4 * e + t] = v[t];
    }
}

__device__ __forceinline__ void transpose_block(const zn_f32x16 &d, float *gt, int lane, float (&b)[16]) {
    float g[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) g[q] = d[q];
    transpose_block(g, gt, lane, b);
}

// LDS: per wave two stages of the operand staged by DMA (up to 64x32) and
// the transposition block; then the workgroup's W2 and gaa2 copies and the
// bias sums' reduction.  107 KB: one workgroup per CU, and the grid is at
// most one per CU.
constexpr int kPairSt = 2048, kPairGt = 32 * kGt;
constexpr int kPairRegion = 2 * kPairSt + kPairGt;
constexpr int kPairRawW = 4 * kPairRegion, kPairRawG = kPairRawW + kRawW, kPairRed = kPairRawG + kRawG;
constexpr int kPairLds = kPairRed + 256;

struct PairWave {
    int lane, wave;
    float *st[2], *gt, *raw_w, *raw_g;
};

__device__ __forceinline__ PairWave pair_wave(float *lds) {
    PairWave w;
    w.lane = threadIdx.x & (kWave - 1);
    w.wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
    float *region = lds + w.wave * kPairRegion;
    w.st[0] = region;
    w.st[1] = region + kPairSt;
    w.gt = region + 2 * kPairSt;
    w.raw_w = lds + kPairRawW;
    w.raw_g = lds + kPairRawG;
    return w;
}

// The end of a tile of FM 32-row accumulator blocks: the four waves'
// partial tiles are added in wave order through LDS and written to C.  TR:
// the accumulators hold the tile transposed (block f covers columns 32f ..
// of C, its rows are C's columns and its columns C's rows).  Thread t writes
// row t / 8 of C (32 rows), 4 FM consecutive columns from 4 FM (t % 8).
template <int FM, bool TR>
__device__ __forceinline__ void pair_finish(const ZnPairGemm &p, float *lds, const zn_f32x16 (&acc)[FM], int m0,
                                            int n0, int wave, int lane) {
    constexpr int kPart = FM * 16 * kWave;
    __syncthreads();  // every wave is done with its staging region
#pragma unroll
    for (int f = 0; f < FM; ++f)
#pragma unroll
        for (int q = 0; q < 16; ++q) lds[wave * kPart + (f * 16 + q) * 64 + lane] = acc[f][q];
    __syncthreads();
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.c, (uint32_t)((p.m - 1) * p.ldc + p.n) * 4u);
    const int t = threadIdx.x;
    const int R = t >> 3;
#pragma unroll
    for (int c = 0; c < 4 * FM; ++c) {
        const int C = 4 * FM * (t & 7) + c;
        const int f = TR ? C >> 5 : 0;
        const int ar = TR ? C & 31 : R, ac = TR ? R : C;  // the element's accumulator row and column
        const int off = (f * 16 + 4 * (ar >> 3) + (ar & 3)) * 64 + 32 * ((ar >> 2) & 1) + ac;
        float x = lds[off];
#pragma unroll
        for (int w = 1; w < 4; ++w) x = x + lds[w * kPart + off];
        bstore(rc, m0 + R < p.m && n0 + C < p.n, (m0 + R) * p.ldc + n0 + C, x);
    }
}

// A wave's K range of a tile whose K is split over four waves: whole
// 32-slices [kbeg, kend), ktiles of them.
struct PairK {
    int kbeg, kend, ktiles;
};

__device__ __forceinline__ PairK pair_k(int k, int wave) {
    const int chunk = ((k + 3) / 4 + 31) / 32 * 32;
    PairK r;
    r.kbeg = min(k, wave * chunk);
    r.kend = min(k, r.kbeg + chunk);
    r.ktiles = (r.kend - r.kbeg + 31) / 32;
    return r;
}

__device__ __forceinline__ int pad32(int x) { return (x + 31) & ~31; }

// grad_x = gaa1 . W1^T on a 32x64 tile (rows m0: batch, columns n0: inputs),
// computed transposed: grad_x^T = W1 . gaa1^T, with A = W1's 64 rows staged
// by DMA (K-contiguous, two 32-row blocks) and B = gaa1^T in registers: the
// grad_h block over this tile's batch rows and the slice's hidden columns is
// already in B's fragment layout, and act1' with h makes it gaa1^T (shared
// by both blocks).  Two slices at a time; the workgroup's copies of W2 (all
// rows) and gaa2 (the tile's rows) and the first two slices are all in
// flight before the first wait.
template <int WD, int ACT1, int ACT2>
__device__ __forceinline__ void pair_tile_nt(const ZnPairBwdArgs &a, const PairSrc &s, float *lds, int wg) {
    const ZnPairGemm &p = a.nt;  // m = batch, n = in, k = hidden; src = W1 [in x hidden]
    typedef DmaStage<64, 32, kWave, true, WD> SW;
    const PairWave w = pair_wave(lds);
    const int tm = wg / p.tiles_n, tn = wg - tm * p.tiles_n;
    const int m0 = tm * 32, n0 = tn * 64;
    const PairK K = pair_k(p.k, w.wave);
    constexpr int RD = WD == 16 ? 3 : 0;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.src, (uint32_t)((p.n - 1) * p.ld + ((p.k + RD) & ~RD)) * 4u);
    const int row = m0 + (w.lane & 31);  // this lane's batch row of gaa1^T
    const int wlen = pad32(s.hidden) * s.out, glen = 32 * s.out;
    const RawPart cw = raw_load<false>(s, s.w2, 0, wlen, s.hidden * s.out);
    const RawPart cg = raw_load<ACT2 != 0>(s, s.gy, m0 * s.out, glen, (s.batch - m0) * s.out);
    float hv[2][16];
    SW::issue(rs, w.st[0], p.ld, n0, K.kbeg, p.n, K.kend, 0, w.lane);
    h_load<WD>(s, row, K.kbeg, w.lane, hv[0]);
    if (K.ktiles > 1) {  // uniform (one slice per wave for hidden <= 128)
        SW::issue(rs, w.st[1], p.ld, n0, K.kbeg + 32, p.n, K.kend, 0, w.lane);
        h_load<WD>(s, row, K.kbeg + 32, w.lane, hv[1]);
    }
    raw_store<false>(s, cw, wlen, w.raw_w);
    raw_store<ACT2 != 0>(s, cg, glen, w.raw_g);
    __syncthreads();  // the workgroup's copies are in LDS
    zn_f32x16 acc[2];
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[f][q] = 0.0f;
    for (int kt = 0; kt < K.ktiles; kt += 2) {
        const int k0 = K.kbeg + kt * 32;
        if (kt > 0) {
            SW::issue(rs, w.st[0], p.ld, n0, k0, p.n, K.kend, 0, w.lane);
            SW::issue(rs, w.st[1], p.ld, n0, k0 + 32, p.n, K.kend, 0, w.lane);
            h_load<WD>(s, row, k0, w.lane, hv[0]);
            h_load<WD>(s, row, k0 + 32, w.lane, hv[1]);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // both slices of W1 are in their stages
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (u == 1 && kt + 1 >= K.ktiles) break;
            float gb[16];
            gaa1_of<ACT1>(hv[u], pair_grad_h(w.raw_w + (k0 + 32 * u) * s.out, w.raw_g, s.out, w.lane), gb);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float fa[2][4];
                read_frags_dma<64, 32, 2, true>(w.st[u], 0, 8 * e, w.lane, fa);
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int f = 0; f < 2; ++f)
                        acc[f] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[f][q], gb[4 * e + q], acc[f], 0, 0, 0);
            }
        }
    }
    pair_finish<2, true>(p, lds, acc, m0, n0, w.wave, w.lane);
}

// grad_w1 = x^T . gaa1 on a 32x32 tile (rows m0: inputs, columns n0:
// hidden), K = batch: A = x's block staged by DMA (X-contiguous), B = gaa1
// from the grad_h block over the slice's batch rows and the tile's hidden
// columns, transposed through LDS into B's fragment layout.  Every tile
// covers every batch row of its columns between its four waves, so the
// tiles of one column share the writes of grad_h and gaa1 (stores along the
// rows, from the transposed blocks): 32-row block b goes out from the tile
// in row b % tiles_m.  The first row's tiles (m0 = 0) also add the columns'
// gaa1 sums into grad_b1: lane (n, h) sums its rows of column n in
// ascending order, and the eight (wave, h) sums are added in that order.
template <int WD, int ACT1, int ACT2>
__device__ __forceinline__ void pair_tile_tn1(const ZnPairBwdArgs &a, const PairSrc &s, float *lds, int wg) {
    const ZnPairGemm &p = a.tn1;  // m = in, n = hidden, k = batch; src = x [batch x in]
    typedef DmaStage<32, 32, kWave, false, WD> SX;
    const PairWave w = pair_wave(lds);
    const int tm = wg / p.tiles_n, tn = wg - tm * p.tiles_n;
    const int m0 = tm * 32, n0 = tn * 32;
    const bool first_row = tm == 0;  // uniform
    const int tiles_m = (p.m + 31) / 32;
    const PairK K = pair_k(p.k, w.wave);
    constexpr int RD = WD == 16 ? 3 : 0;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.src, (uint32_t)((p.k - 1) * p.ld + ((p.m + RD) & ~RD)) * 4u);
    const int wlen = 32 * s.out, glen = pad32(s.batch) * s.out;
    const RawPart cw = raw_load<false>(s, s.w2, n0 * s.out, wlen, (s.hidden - n0) * s.out);
    const RawPart cg = raw_load<ACT2 != 0>(s, s.gy, 0, glen, s.batch * s.out);
    float hv[2][16];
    SX::issue(rs, w.st[0], p.ld, m0, K.kbeg, p.m, K.kend, 0, w.lane);
    SX::issue(rs, w.st[1], p.ld, m0, K.kbeg + 32, p.m, K.kend, 0, w.lane);
    h_load<WD>(s, K.kbeg + (w.lane & 31), n0, w.lane, hv[0]);
    h_load<WD>(s, K.kbeg + 32 + (w.lane & 31), n0, w.lane, hv[1]);
    // the first row's old bias gradient, read early so that its latency hides
    const int t = threadIdx.x;
    const bool bias_lane = first_row && t < 32 && n0 + t < s.hidden;
    const float b1_old = bias_lane ? a.grad_b1[n0 + t] : 0.0f;
    raw_store<false>(s, cw, wlen, w.raw_w);
    raw_store<ACT2 != 0>(s, cg, glen, w.raw_g);
    __syncthreads();  // the workgroup's copies are in LDS
    const int n = w.lane & 31, h = w.lane >> 5;
    const int col = n0 + n;
    const int cells = s.batch * s.hidden;
    const __amdgpu_buffer_rsrc_t rgh = make_rsrc(a.grad_h, (uint32_t)cells * 4u);
    const __amdgpu_buffer_rsrc_t rga = make_rsrc(a.gaa1, (uint32_t)cells * 4u);
    float sum = 0.0f;
    zn_f32x16 acc;
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[q] = 0.0f;
    for (int kt = 0; kt < K.ktiles; kt += 2) {
        const int k0 = K.kbeg + kt * 32;
        if (kt > 0) {
            SX::issue(rs, w.st[0], p.ld, m0, k0, p.m, K.kend, 0, w.lane);
            SX::issue(rs, w.st[1], p.ld, m0, k0 + 32, p.m, K.kend, 0, w.lane);
            h_load<WD>(s, k0 + (w.lane & 31), n0, w.lane, hv[0]);
            h_load<WD>(s, k0 + 32 + (w.lane & 31), n0, w.lane, hv[1]);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // both slices of x are in their stages
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (u == 1 && kt + 1 >= K.ktiles) break;
            const int r0 = k0 + 32 * u;
            const zn_f32x16 d = pair_grad_h(w.raw_w, w.raw_g + r0 * s.out, s.out, w.lane);
            float g[16], gb[16];
            gaa1_of<ACT1>(hv[u], d, g);
            transpose_block(g, w.gt, w.lane, gb);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float fa[1][4];
                read_frags_dma<32, 32, 1, false>(w.st[u], 0, 8 * e, w.lane, fa);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[0][q], gb[4 * e + q], acc, 0, 0, 0);
            }
            if ((r0 >> 5) % tiles_m == tm) {  // uniform: this tile writes the block
                float dc[16];
                transpose_block(d, w.gt, w.lane, dc);
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int r = r0 + acc_row(q, h);
                    const bool ok = r < s.batch && col < s.hidden;
                    bstore(rgh, ok, r * s.hidden + col, dc[q]);
                    bstore(rga, ok, r * s.hidden + col, gb[q]);
                }
            }
            if (first_row) {  // uniform
#pragma unroll
                for (int q = 0; q < 16; ++q) sum = sum + gb[q];  // +0 outside the batch or the columns
            }
        }
    }
    if (first_row) {  // uniform; the LDS below is outside every wave's region
        float *red = lds + kPairRed;
        red[w.wave * 64 + w.lane] = sum;
        __syncthreads();
        if (bias_lane) {
            float total = red[t];
            for (int k = 1; k < 8; ++k) total = total + red[(k >> 1) * 64 + (k & 1) * 32 + t];
            a.grad_b1[n0 + t] = b1_old + total;
        }
    }
    zn_f32x16 accs[1] = {acc};
    pair_finish<1, false>(p, lds, accs, m0, n0, w.wave, w.lane);
}

// grad_w2 = h^T . gaa2 on a 32x32 tile (rows m0: hidden, columns: the head,
// zero past out), K = batch: A = h's block staged by DMA, B = gaa2 read
// from the workgroup's copy in its fragment layout.  The first tile (m0 = 0)
// also writes gaa2 from its copy and adds its column sums into grad_b2:
// thread t takes column t % 16 and rows t / 16 + 16i in ascending order,
// and the 16 threads' sums of a column are added in thread order.
template <int WD, int ACT2>
__device__ __forceinline__ void pair_tile_tn2(const ZnPairBwdArgs &a, const PairSrc &s, float *lds, int wg) {
    const ZnPairGemm &p = a.tn2;  // m = hidden, n = out, k = batch; src = h [batch x hidden]
    typedef DmaStage<32, 32, kWave, false, WD> SH;
    const PairWave w = pair_wave(lds);
    const int m0 = wg * 32;
    const PairK K = pair_k(p.k, w.wave);
    constexpr int RD = WD == 16 ? 3 : 0;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.src, (uint32_t)((p.k - 1) * p.ld + ((p.m + RD) & ~RD)) * 4u);
    const int j = w.lane & 31, h = w.lane >> 5;
    const int glen = pad32(s.batch) * s.out;
    const RawPart cg = raw_load<ACT2 != 0>(s, s.gy, 0, glen, s.batch * s.out);
    const bool bias_lane = wg == 0 && (int)threadIdx.x < s.out;
    const float b2_old = bias_lane ? a.grad_b2[threadIdx.x] : 0.0f;  // read early: its latency hides
    SH::issue(rs, w.st[0], p.ld, m0, K.kbeg, p.m, K.kend, 0, w.lane);
    SH::issue(rs, w.st[1], p.ld, m0, K.kbeg + 32, p.m, K.kend, 0, w.lane);
    raw_store<ACT2 != 0>(s, cg, glen, w.raw_g);
    __syncthreads();  // the workgroup's copy is in LDS
    if (wg == 0) {  // uniform: gaa2 and grad_b2
        const int t = threadIdx.x, c = t & 15;
        const __amdgpu_buffer_rsrc_t rg = make_rsrc(a.gaa2, (uint32_t)(s.batch * s.out) * 4u);
        float sum = 0.0f;
        for (int r = t >> 4; r < s.batch; r += 16) {
            const float g = c < s.out ? w.raw_g[r * s.out + min(c, s.out - 1)] : 0.0f;
            bstore(rg, c < s.out, r * s.out + c, g);
            sum = sum + g;
        }
        float *red = lds + kPairRed;
        red[t] = sum;
        __syncthreads();
        if (bias_lane) {
            float total = red[t];
            for (int k = 1; k < 16; ++k) total = total + red[k * 16 + t];
            a.grad_b2[t] = b2_old + total;
        }
    }
    zn_f32x16 acc;
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[q] = 0.0f;
    const int jc = min(j, s.out - 1);
    for (int kt = 0; kt < K.ktiles; kt += 2) {
        const int k0 = K.kbeg + kt * 32;
        if (kt > 0) {
            SH::issue(rs, w.st[0], p.ld, m0, k0, p.m, K.kend, 0, w.lane);
            SH::issue(rs, w.st[1], p.ld, m0, k0 + 32, p.m, K.kend, 0, w.lane);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // both slices of h are in their stages
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (u == 1 && kt + 1 >= K.ktiles) break;
            float gb[16];
#pragma unroll
            for (int q = 0; q < 16; ++q)
                gb[q] = j < s.out ? w.raw_g[(k0 + 32 * u + acc_row(q, h)) * s.out + jc] : 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float fa[1][4];
                read_frags_dma<32, 32, 1, false>(w.st[u], 0, 8 * e, w.lane, fa);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[0][q], gb[4 * e + q], acc, 0, 0, 0);
            }
        }
    }
    zn_f32x16 accs[1] = {acc};
    pair_finish<1, false>(p, lds, accs, m0, 0, w.wave, w.lane);
}

// Each workgroup type computes its own view of the inputs, so that no
// value stays live across the branches.
template <int WD, int ACT1, int ACT2>
__device__ __forceinline__ void pair_backward(const ZnPairBwdArgs &a, float *lds) {
    const int b = blockIdx.x;
    const int b1 = b - a.wg_nt, b2 = b1 - a.wg_tn1;
    if (b1 < 0)
        pair_tile_nt<WD, ACT1, ACT2>(a, pair_src(a), lds, b);
    else if (b2 < 0)
        pair_tile_tn1<WD, ACT1, ACT2>(a, pair_src(a), lds, b1);
    else
        pair_tile_tn2<WD, ACT2>(a, pair_src(a), lds, b2);
}

}  // namespace

// zn_dense_pair_fwd[_v]: _v stages x and W1 with 16-byte loads.
#define ZN_PAIR_FWD_KERNEL(SUFFIX, W)                                                            \
    extern "C" __global__ __launch_bounds__(kPairFwdWaves * 64, 1) void zn_dense_pair_fwd##SUFFIX(ZnPairFwdArgs a) { \
        __shared__ __attribute__((aligned(1024))) float lds[4 * 8 * 32 * 32];                     \
        switch (a.l1.act) {                                                                      \
        case 1: pair_forward<W, 1>(a, lds); break;                                               \
        case 2: pair_forward<W, 2>(a, lds); break;                                               \
        case 3: pair_forward<W, 3>(a, lds); break;                                               \
        default: pair_forward<W, 0>(a, lds); break;                                              \
        }                                                                                        \
    }
ZN_PAIR_FWD_KERNEL(_v, 16)
ZN_PAIR_FWD_KERNEL(, 4)

// zn_dense_pair_bwd_<act1><head>[_v]: one kernel per activation of the
// lower layer (0-3) and kind of head (0: linear, 1: non-linear, whose
// derivative reads y), so that each is register-allocated on its own (one
// kernel holding every combination spilled thousands of scalar registers).
// _v stages W1, x and h with 16-byte loads.  107 KB of LDS, one workgroup
// per CU.
#define ZN_PAIR_BWD_KERNEL(A1, A2, SUFFIX, WD)                                                   \
    extern "C" __global__ __launch_bounds__(256, 1) void zn_dense_pair_bwd_##A1##A2##SUFFIX(ZnPairBwdArgs a) { \
        __shared__ __attribute__((aligned(1024))) float lds[kPairLds];                           \
        pair_backward<WD, A1, A2>(a, lds);                                                       \
    }
#define ZN_PAIR_BWD_KERNELS(A1)                                                                  \
    ZN_PAIR_BWD_KERNEL(A1, 0, _v, 16)                                                            \
    ZN_PAIR_BWD_KERNEL(A1, 1, _v, 16)                                                            \
    ZN_PAIR_BWD_KERNEL(A1, 0, , 4)                                                               \
    ZN_PAIR_BWD_KERNEL(A1, 1, , 4)
ZN_PAIR_BWD_KERNELS(0)
ZN_PAIR_BWD_KERNELS(1)
ZN_PAIR_BWD_KERNELS(2)
ZN_PAIR_BWD_KERNELS(3)
