// zn_hip.cpp -- host runtime of the MI355X fp32 GEMM backend (C ABI in
// include/zn_hip.h).
//
// Replaces, for the GEMM path, the reference's CUDA driver binding, NVRTC
// and device context (src/cuda_driver.zig, src/cuda_nvrtc.zig,
// src/cuda_context.zig) and the CudaBackend GEMM wrappers (src/cuda.zig).
// Design:
//  * one context = one device + one HIP stream + the four offline-built
//    gfx950 code objects (zn_gemm_gfx950.hsaco, zn_conv_gfx950.hsaco,
//    zn_elementwise_gfx950.hsaco, zn_attention_gfx950.hsaco) and the fused
//    two-layer Dense kernels (zn_mlp_gfx950.hsaco), loaded with
//    hipModuleLoad; no runtime compilation, no CPU fallback;
//  * a size-bucketed device-buffer cache for the host-slice entry points
//    (the role of the pow2 pool in src/cuda_context.zig:773-852);
//  * the launch policy (tile choice, raster, vector-load eligibility) lives
//    here, so it is testable without touching device code.
#include <hip/hip_runtime.h>

#include <dlfcn.h>

#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <condition_variable>
#include <map>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "../../../include/zn_hip.h"
#include "../zn_kernel_args.h"

// Scratch of zn_hip_sgemm_noalloc: the split-K partial sums of a GEMM whose
// caller cannot allocate.  One copy per device, held until the process ends.
// In host code `scratch` only names the symbol; its device address on each
// device comes from hipGetSymbolAddress (resolve_scratch below), and only
// that address is ever passed to a kernel.
constexpr size_t kScratchBytes = (size_t)64 << 20;
constexpr int64_t kCounterSlots = 4096;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

// Macro tiles of the GEMM code object (kernels/gemm_f32.hip).
enum Tile { kTileX = 0, kTileL, kTileN, kTileM, kTileS, kTileR, kTileH, kTileW, kNumTiles };
struct TileShape {
    int bm, bn, bk, threads;
    const char *suffix;
    bool conv;        // the convolution code object has kernels for it
    bool persistent;  // zn_sgemmp_<layout>_<suffix>_v exists
    bool plain;       // a 4-byte-staging kernel (no _v suffix) exists
};
constexpr TileShape kTiles[kNumTiles] = {{256, 128, 16, 512, "x", true, true, true},
                                         {128, 128, 16, 256, "l", true, true, true},
                                         {128, 64, 16, 128, "n", true, true, true},
                                         {64, 64, 32, 256, "m", true, true, true},
                                         {32, 32, 32, 64, "s", true, false, true},
                                         {128, 128, 32, 512, "r", false, false, true},
                                         {64, 64, 16, 256, "h", false, false, true},
                                         {256, 256, 16, 512, "w", false, false, false}};
constexpr const char *kLayoutName[3] = {"nn", "nt", "tn"};

enum EltKernel { kFill, kCopy, kAddBias, kActFwd, kActBwd, kAccBias, kIm2col, kSoftmax, kCol2im, kRowSum, kDenseGrad, kRegroup, kPack, kToNhwc, kHold, kNumElt };
constexpr const char *kEltName[kNumElt] = {"zn_fill_f32",        "zn_copy_f32", "zn_add_bias",
                                           "zn_activation_forward", "zn_activation_backward",
                                           "zn_accumulate_bias", "zn_im2col",   "zn_softmax_rows",
                                           "zn_col2im",          "zn_row_sum",  "zn_dense_grad_prologue",
                                           "zn_weight_regroup", "zn_pack_rows", "zn_nchw_to_nhwc",
                                           "zn_hold_stream"};

constexpr const char *kGemmObject = "zn_gemm_gfx950.hsaco";
constexpr const char *kConvObject = "zn_conv_gfx950.hsaco";
constexpr const char *kEltObject = "zn_elementwise_gfx950.hsaco";
constexpr const char *kMlpObject = "zn_mlp_gfx950.hsaco";
constexpr const char *kAttnObject = "zn_attention_gfx950.hsaco";
// Fused attention kernels by padded head dim (zn_attention_d<dim>[_v]).
constexpr int kAttnDims[3] = {32, 64, 128};
constexpr int kAttnQueries = 128;  // queries per workgroup (4 waves x 32)

struct ScratchDevice;

}  // namespace

// Host memcpy split over a few persistent threads (the caller takes one
// part).  One host thread drives a context, so one copy runs at a time.
struct HostCopier {
    std::vector<std::thread> workers;
    std::mutex mu;
    std::condition_variable job_cv, done_cv;
    char *dst = nullptr;
    const char *src = nullptr;
    size_t bytes = 0;
    uint64_t generation = 0;
    int pending = 0;
    bool stop = false;

    explicit HostCopier(int threads) {
        for (int i = 0; i < threads; ++i) workers.emplace_back([this, i] { run(i + 1); });
    }
    ~HostCopier() {
        {
            std::lock_guard<std::mutex> g(mu);
            stop = true;
        }
        job_cv.notify_all();
        for (auto &t : workers) t.join();
    }
    // Part `part` of `parts` equal 64-byte-aligned slices of the current job.
    void slice(int part, int parts) const {
        const size_t per = ((bytes + parts - 1) / parts + 63) & ~(size_t)63;
        const size_t begin = std::min(bytes, per * part), end = std::min(bytes, begin + per);
        if (end > begin) std::memcpy(dst + begin, src + begin, end - begin);
    }
    void run(int part) {
        uint64_t seen = 0;
        for (;;) {
            std::unique_lock<std::mutex> lk(mu);
            job_cv.wait(lk, [&] { return stop || generation != seen; });
            if (stop) return;
            seen = generation;
            lk.unlock();
            slice(part, (int)workers.size() + 1);
            lk.lock();
            if (--pending == 0) done_cv.notify_one();
        }
    }
    void copy(void *d, const void *s, size_t n) {
        if (workers.empty() || n < ((size_t)1 << 20)) {
            std::memcpy(d, s, n);
            return;
        }
        {
            std::lock_guard<std::mutex> g(mu);
            dst = (char *)d;
            src = (const char *)s;
            bytes = n;
            pending = (int)workers.size();
            ++generation;
        }
        job_cv.notify_all();
        slice(0, (int)workers.size() + 1);
        std::unique_lock<std::mutex> lk(mu);
        done_cv.wait(lk, [&] { return pending == 0; });
    }
};

struct zn_ctx {
    int device = -1;
    hipStream_t stream = nullptr;
    hipModule_t gemm_module = nullptr;
    hipModule_t conv_module = nullptr;
    hipModule_t elt_module = nullptr;
    hipModule_t attn_module = nullptr;
    hipModule_t mlp_module = nullptr;
    hipFunction_t pair_fwd[2] = {};            // fused two-layer Dense forward [16-byte staging]
    int pair_fwd_threads[2] = {};              // its workgroup size (the kernel's launch bounds)
    hipFunction_t pair_bwd[4][2][2] = {};      // fused two-layer Dense backward [lower act][non-linear head][16-byte]
    hipFunction_t attn[3][2] = {};             // fused attention [head dim 32/64/128][16-byte I/O]
    hipFunction_t gemm[3][kNumTiles][3] = {};  // [layout][tile][staging: 4-byte, 16-byte, 16-byte unaligned (r only)]
    int gemm_threads[3][kNumTiles][3] = {};    // their workgroup sizes (the kernels' launch bounds)
    hipFunction_t conv[kNumTiles][2][2] = {};  // implicit-GEMM convolution [tile][16-byte W rows][4-pixel gather]
    hipFunction_t convt[kNumTiles][2] = {};    // stride-1 transposed convolution [tile][16-byte W' rows]
    int convt_occ[kNumTiles][2] = {};          // their resident workgroups per CU
    hipFunction_t convw[kNumTiles][2] = {};    // implicit weight gradient [tile][16-byte grad_output rows]
    hipFunction_t gemmq[3][3][2] = {};         // [layout][q4, q4m, q8][16-byte]: 16x16 wave-split tiles
    int gemmq_threads[3][3][2] = {};           // their workgroup sizes (the kernels' launch bounds)
    hipFunction_t gemmks[3][2] = {};           // [layout][16-byte]: 32x32 wave-split tiles with K split over workgroups too
    hipFunction_t dense_bwd[2] = {};           // grouped Dense backward GEMMs [16-byte staging]
    hipFunction_t dense_bwd_k[2] = {};         // the same on 32x32 tiles with K split over 4 waves [16-byte]
    hipFunction_t convf[kNumTiles][2] = {};    // convolution forward on NHWC [tile][16-byte W rows]
    hipFunction_t convwn[kNumTiles][2] = {};   // weight gradient on NHWC [tile][16-byte grad_output rows]
    hipFunction_t gemmp[3][kNumTiles] = {};    // persistent plain GEMM, 16-byte staging [layout][tile] (not s)
    hipFunction_t gemmk[3][2][2] = {};         // intra-workgroup split-K, 32x32 tiles [layout][4 or 8 waves][16-byte]
    int gemmp_occ[3][kNumTiles] = {};          // its resident workgroups per CU
    hipFunction_t gemmpd[3] = {};              // [layout]: persistent 128x128 with deferred stores
    hipFunction_t gemmpd4[3] = {};             // [layout]: the same for K of exactly 4 slices
    int gemmpd_occ[3] = {};
    int gemmpd_threads[3] = {};                // its workgroup size (the kernel's launch bound)
    hipFunction_t splitk_reduce = nullptr;
    // Split-K workspace (partial sums), grown on demand and kept until destroy.
    float *ws = nullptr;
    size_t ws_bytes = 0;
    int32_t *counters = nullptr;  // kCounterSlots arrival counters, kCounterStride ints apart, zero between launches
    hipFunction_t elt[kNumElt] = {};
    int last_hip_error = 0;
    // Graph capture (zn_hip_graph_begin .. _end): leased buffers go to
    // `captured` instead of back to the pool and become the graph's.
    bool capturing = false;
    std::vector<std::pair<void *, size_t>> captured;
    std::vector<zn_graph *> graphs;   // live graphs, destroyed with the context
    std::vector<void *> retired_ws;   // workspaces a live graph may still reference
    int forced_tile = -1;    // ZN_TILE_AUTO
    int forced_splits = 0;   // 0: the split-K policy decides
    int forced_persistent = -1;  // -1: the policy decides; 0: never; 1: whenever eligible
    int forced_wave_split = -1;  // -1: the policy decides; 0: never; 4 or 8: that many waves whenever eligible
    zn_device_info info = {};
    // Cached device buffers for the host-slice entry points, keyed by
    // power-of-two byte size.
    std::map<size_t, std::vector<void *>> pool;
    // Host-slice copies of 4 MiB and more go through two pinned staging
    // buffers (hipHostMalloc, created on first use): a threaded host memcpy
    // fills or drains one while the DMA engine moves the other.  Pageable
    // copies ran at 21 GB/s H2D and 15 GB/s D2H on MI355X, pinned ones at 57.
    float *pinned[2] = {};
    hipEvent_t pinned_done[2] = {};
    std::unique_ptr<HostCopier> copier;
    // Pipelined host-slice GEMMs (created on first use): an upload and a
    // download stream, a second pinned ring for downloads, and per-chunk
    // events (A chunk uploaded, C chunk computed; by chunk parity).
    hipStream_t up = nullptr, down = nullptr;
    float *pinned_out[2] = {};
    hipEvent_t pinned_out_done[2] = {};
    hipEvent_t chunk_in[2] = {}, chunk_out[2] = {};
    hipEvent_t entry = nullptr;
    // This device's copy of `scratch` (resolved at create), its ordering
    // state and, while zn_hip_sgemm_noalloc runs, the flag that routes its
    // split-K partial sums there and turns operand packing off.
    float *scratch = nullptr;
    ScratchDevice *scratch_dev = nullptr;
    int scratch_status = ZN_OK;
    bool no_alloc = false;
};

struct zn_event {
    hipEvent_t ev = nullptr;
};

struct zn_graph {
    zn_ctx *ctx = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<std::pair<void *, size_t>> buffers;  // leased during capture
};

namespace {

int fail_hip(zn_ctx *ctx, hipError_t e, int status = ZN_ERR_HIP) {
    if (ctx) ctx->last_hip_error = (int)e;
    return status;
}

#define ZN_HIP_TRY(ctx, expr)                          \
    do {                                               \
        hipError_t zn_e_ = (expr);                     \
        if (zn_e_ != hipSuccess) return fail_hip((ctx), zn_e_); \
    } while (0)

bool mul_ok(size_t a, size_t b, size_t *out) {
    if (a != 0 && b > SIZE_MAX / a) return false;
    *out = a * b;
    return true;
}

// Host-side check of a code object before the runtime sees it: a clang
// offload bundle (what `hipcc --genco` writes) with an amdgcn gfx950 entry,
// or a bare ELF, whose AMDGPU ELF header and program and section header
// tables lie inside the file.  A missing, truncated or foreign file is then
// ZN_ERR_CODE_OBJECT without ever reaching hipModuleLoad.
constexpr uint16_t kEmAmdgpu = 224;          // ELF e_machine of AMDGPU code objects
constexpr uint32_t kMachGfx950 = 0x04f;      // e_flags & 0xff (EF_AMDGPU_MACH) for gfx950

template <typename T>
T load_le(const unsigned char *p) {
    T v;
    std::memcpy(&v, p, sizeof(T));
    return v;
}

bool amdgpu_elf_ok(const unsigned char *p, size_t n) {
    if (n < 64 || std::memcmp(p, "\x7f" "ELF", 4) != 0 || p[4] != 2 || p[5] != 1) return false;  // 64-bit, LE
    if (load_le<uint16_t>(p + 18) != kEmAmdgpu) return false;
    if ((load_le<uint32_t>(p + 48) & 0xff) != kMachGfx950) return false;
    const uint64_t phoff = load_le<uint64_t>(p + 32), shoff = load_le<uint64_t>(p + 40);
    const uint64_t ph = (uint64_t)load_le<uint16_t>(p + 54) * load_le<uint16_t>(p + 56);
    const uint64_t sh = (uint64_t)load_le<uint16_t>(p + 58) * load_le<uint16_t>(p + 60);
    return phoff <= n && ph <= n - phoff && shoff <= n && sh <= n - shoff;
}

bool code_object_ok(const std::string &path) {
    FILE *f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    std::vector<unsigned char> buf;
    unsigned char chunk[1 << 16];
    size_t got;
    while ((got = std::fread(chunk, 1, sizeof(chunk), f)) > 0) buf.insert(buf.end(), chunk, chunk + got);
    std::fclose(f);
    const size_t n = buf.size();
    const unsigned char *p = buf.data();
    static const char kBundle[] = "__CLANG_OFFLOAD_BUNDLE__";
    const size_t magic = sizeof(kBundle) - 1;
    if (n < magic || std::memcmp(p, kBundle, magic) != 0) return amdgpu_elf_ok(p, n);
    if (n < magic + 8) return false;
    const uint64_t entries = load_le<uint64_t>(p + magic);
    size_t at = magic + 8;
    bool found = false;
    for (uint64_t i = 0; i < entries; ++i) {
        if (n - at < 24) return false;
        const uint64_t off = load_le<uint64_t>(p + at), size = load_le<uint64_t>(p + at + 8);
        const uint64_t tlen = load_le<uint64_t>(p + at + 16);
        at += 24;
        if (tlen > n - at || off > n || size > n - off) return false;
        const std::string triple((const char *)p + at, (size_t)tlen);
        at += (size_t)tlen;
        if (triple.find("amdgcn") != std::string::npos) {
            if (triple.find("gfx950") == std::string::npos || !amdgpu_elf_ok(p + off, (size_t)size)) return false;
            found = true;
        }
    }
    return found;
}

// Directory holding this shared library (the default code-object location).
std::string library_dir() {
    Dl_info info;
    if (dladdr(reinterpret_cast<void *>(&zn_hip_abi_version), &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        const size_t slash = p.find_last_of('/');
        if (slash != std::string::npos) return p.substr(0, slash);
    }
    return ".";
}

int select_device(zn_ctx *ctx) {
    ZN_HIP_TRY(ctx, hipSetDevice(ctx->device));
    return ZN_OK;
}

// One device's `scratch`: its device address, resolved once with that device
// current and kept for the process (each device holds its own copy at its
// own address), and the ordering of the calls that use it.  Every context on
// the device shares it.  A call queues its kernels under `use`, after a wait
// for `done` when another context recorded it last, and records `done`
// behind them, so calls from different contexts (streams) run one after the
// other on the device instead of overlapping on the one array.
struct ScratchDevice {
    std::mutex use;
    bool resolved = false;
    float *ptr = nullptr;
    hipEvent_t done = nullptr;     // recorded behind the last call's kernels
    bool recorded = false;
    const zn_ctx *owner = nullptr;  // the context that recorded `done` last (null: gone)
};
std::mutex g_scratch_mu;
std::map<int, ScratchDevice> g_scratch;  // by device; the map never moves an entry

// Only a success is kept: after a failure the next context created on the
// device tries again.
int resolve_scratch(zn_ctx *ctx) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ScratchDevice &s = g_scratch[ctx->device];
    if (!s.resolved) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e == hipSuccess && !p) e = hipErrorInvalidSymbol;
        hipEvent_t ev = nullptr;
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            ctx->scratch = nullptr;
            ctx->scratch_dev = nullptr;
            ctx->scratch_status = e == hipErrorOutOfMemory ? ZN_ERR_OOM : ZN_ERR_HIP;
            ctx->last_hip_error = (int)e;
            return ctx->scratch_status;
        }
        s.ptr = static_cast<float *>(p);
        s.done = ev;
        s.resolved = true;
    }
    ctx->scratch = s.ptr;
    ctx->scratch_dev = &s;
    ctx->scratch_status = ZN_OK;
    return ZN_OK;
}

// A context that goes away no longer owns the device's last scratch record
// (its stream was drained before this runs).
void forget_scratch_owner(zn_ctx *ctx) {
    if (!ctx->scratch_dev) return;
    std::lock_guard<std::mutex> lock(ctx->scratch_dev->use);
    if (ctx->scratch_dev->owner == ctx) ctx->scratch_dev->owner = nullptr;
}

// Marks a context as running zn_hip_sgemm_noalloc for one call.
struct NoAllocScope {
    zn_ctx *ctx;
    explicit NoAllocScope(zn_ctx *c) : ctx(c) { ctx->no_alloc = true; }
    ~NoAllocScope() { ctx->no_alloc = false; }
};

size_t bucket_of(size_t bytes) {
    size_t b = 256;
    while (b < bytes) b <<= 1;
    return b;
}

int pool_get(zn_ctx *ctx, size_t bytes, float **out) {
    const size_t b = bucket_of(bytes ? bytes : 4);
    auto &list = ctx->pool[b];
    if (!list.empty()) {
        *out = static_cast<float *>(list.back());
        list.pop_back();
        return ZN_OK;
    }
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, b);
    if (e != hipSuccess) {
        // release cached buffers (after the stream drains: queued kernels may
        // still use buffers returned to the cache) and retry once
        (void)hipGetLastError();
        if (ctx->capturing) return fail_hip(ctx, e, ZN_ERR_OOM);  // no stream sync under capture
        (void)hipStreamSynchronize(ctx->stream);
        for (auto &kv : ctx->pool)
            for (void *q : kv.second) (void)hipFree(q);
        ctx->pool.clear();
        e = hipMalloc(&p, b);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return fail_hip(ctx, e, ZN_ERR_OOM);
        }
    }
    *out = static_cast<float *>(p);
    return ZN_OK;
}

void pool_put(zn_ctx *ctx, float *p, size_t bytes) {
    if (!p) return;
    if (ctx->capturing)
        ctx->captured.emplace_back(p, bucket_of(bytes ? bytes : 4));  // the graph keeps using it
    else
        ctx->pool[bucket_of(bytes ? bytes : 4)].push_back(p);
}

// Make the split-K workspace at least `bytes` long.  Growing waits for the
// stream first, because queued kernels may still use the old buffer.
int ensure_workspace(zn_ctx *ctx, size_t bytes) {
    if (ctx->ws_bytes >= bytes) return ZN_OK;
    if (ctx->capturing) return ZN_ERR_INVALID_ARG;  // no sync under capture: the GEMM runs unsplit
    size_t want = ctx->ws_bytes ? ctx->ws_bytes : ((size_t)1 << 22);
    while (want < bytes) want <<= 1;
    ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->ws && !ctx->graphs.empty())
        ctx->retired_ws.push_back(ctx->ws);  // a live graph may reference it
    else if (ctx->ws)
        (void)hipFree(ctx->ws);
    ctx->ws = nullptr;
    ctx->ws_bytes = 0;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail_hip(ctx, e, ZN_ERR_OOM);
    }
    ctx->ws = static_cast<float *>(p);
    ctx->ws_bytes = want;
    return ZN_OK;
}

// RAII lease of pooled staging buffers (returned to the cache on scope exit).
struct Lease {
    zn_ctx *ctx;
    float *ptr = nullptr;
    size_t bytes = 0;
    explicit Lease(zn_ctx *c) : ctx(c) {}
    int get(size_t n_floats) {
        bytes = n_floats * sizeof(float);
        return pool_get(ctx, bytes, &ptr);
    }
    ~Lease() { pool_put(ctx, ptr, bytes); }
};

// Every kernel takes one argument block by value; the runtime copies it into
// the kernarg segment using the kernel's own metadata.
int launch(zn_ctx *ctx, hipFunction_t f, unsigned gx, unsigned gy, unsigned threads, void *args, unsigned gz = 1) {
    void *params[] = {args};
    hipError_t e = hipModuleLaunchKernel(f, gx, gy, gz, threads, 1, 1, 0, ctx->stream, params, nullptr);
    if (e != hipSuccess) return fail_hip(ctx, e, ZN_ERR_LAUNCH);
    return ZN_OK;
}

// ------------------------------------------------------------ GEMM policy
int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// K slices for the 128x128 BK 32 tile (one workgroup per CU): the most, up
// to 16 and with at least 768 of K each, that keep tiles x slices within one
// round of workgroups.
int64_t round_splits(int64_t tiles, int64_t k, int64_t cus) {
    const int64_t max_s = std::max<int64_t>(1, std::min<int64_t>(16, k / 768));
    int64_t s = 1;
    while (s < max_s && tiles * (s + 1) <= cus) ++s;
    return s;
}

// The device's compute units, or MI355X's 256 when the query gave none.
int64_t cus_now(const zn_ctx *ctx) { return ctx->info.compute_units > 0 ? ctx->info.compute_units : 256; }

// Tile choice, from measurements on MI355X (256 CUs, per-launch times from
// graph replays): the largest tiles win once they give every CU two or more
// workgroups; below that, 64x64 tiles (4 waves) are the fastest down to the
// smallest problems and for N <= 64 (C5 P.V: 169 us against 184 us for
// 128x64), except for exactly one round of 128x128 tiles (below); 32x32 and
// 128x64 tiles never beat them and are left to explicit selection.  A tile
// whose padding wastes more than a quarter of its MFMA work (for example
// 256-row tiles over M = 128) is skipped for the next smaller one.
// A gathered (implicit convolution) operand costs more per staged element, so
// the larger l tile, which reuses each staged element over 128 rows, pays
// off from 2 instead of 4 tiles per CU (C5 conv: l 221 us, m 227 us).
Tile choose_tile(const zn_ctx *ctx, int64_t m, int64_t n, int64_t k, int64_t batch, bool gathered = false,
                 bool wide_ok = false) {
    const int64_t cus = cus_now(ctx);
    auto tiles = [&](Tile t) { return cdiv(m, kTiles[t].bm) * cdiv(n, kTiles[t].bn) * batch; };
    auto useful = [&](Tile t) { return 4 * m * n * batch >= 3 * tiles(t) * kTiles[t].bm * kTiles[t].bn; };
    // 256x256 (16-byte staging only, one workgroup per CU): long K and whole
    // rounds of tiles, the last at least 80% full (8192^3 NN 141.7 -> 145.4
    // TFLOP/s, 4096^3 125.5 -> 133.7 against 256x128; a ragged last round
    // would leave CUs idle for a whole 256x256 tile)
    if (wide_ok && k >= 512 && tiles(kTileW) >= cus && useful(kTileW) &&
        5 * tiles(kTileW) >= 4 * cdiv(tiles(kTileW), cus) * cus)
        return kTileW;
    // short K: a tile's epilogue outweighs its K walk, and the smaller l tile
    // overlaps them better (C5 QK^T, K = 64: l 242 us, x 252 us, round-robin
    // A/B); up to K = 128 its persistent kernels take the problem
    if (k <= 128 && tiles(kTileL) >= 2 * cus && useful(kTileL)) return kTileL;
    // Whole rounds of 128x128 tiles (every round at least 85% full on
    // average) on the register-staged 128x128 loop, one workgroup of 8 waves
    // per CU: 4096x2048x1024 NN 140.3 -> 126.3 us (against 64x64), 8192x3072
    // x 1024 390.7 -> 369.1 us and 6144x4096x1024 390.6 -> 368.8 us (against
    // 256x128 and 128x128 on 4 waves), 4096x2048x256 49.3 -> 38.2 us,
    // 3840x2048x1024 (1.9 rounds) 138.7 -> 126.4 us; 2.5 rounds stay on
    // 64x64 (5120x2048x1024: 172.9 against 184.7 us).  16-byte rows only:
    // 4-byte rows run the 128x128 tile on the pinned loop, kept to one round.
    if (wide_ok && !gathered && tiles(kTileR) > cus && useful(kTileR) &&
        20 * tiles(kTileR) >= 17 * cdiv(tiles(kTileR), cus) * cus)
        return kTileR;
    if (tiles(kTileX) >= 2 * cus && useful(kTileX)) return kTileX;
    if (tiles(kTileL) >= (gathered ? 2 : 4) * cus && useful(kTileL)) return kTileL;
    // One round of 128x128 tiles (at least 85% of the CUs, counting K slices
    // of at least 768): one workgroup of 8 waves per CU on the three-stage
    // 128x128 loop (against the 64x64 tiles: 4096x1024x1024 NT 74.0 -> 70.4
    // us, 2048^3 NN 139.8 -> 135.5 us, 2048x2048x4096 TN 277.1 -> 257.8 us,
    // 2048x1792x1024 NN (224 tiles) 72.5 -> 70.8 us; C3 dW 1024x1024x4096 TN
    // in 4 slices 76.7 -> 74.5 us, 1024x1024x8192 TN 144.6 -> 137.5 us).
    // Fewer tiles stay on 64x64 (2048x1536x1024, 192 tiles: 56.0 us against
    // 70.4 us).
    if (!gathered && tiles(kTileR) <= cus && useful(kTileR) &&
        20 * tiles(kTileR) * round_splits(tiles(kTileR), k, cus) >= 17 * cus)
        return kTileR;
    // 64x64: BK 32 while the tiles fit one round at its three workgroups per
    // CU, BK 16 (six per CU) beyond (3072x2048x1024 NN: 108.8 -> 106.3 us,
    // 4096x1024x777 NN: 65.4 -> 60.1 us; 1024^3 stays at 23.9 us on BK 32,
    // 29.9 us on BK 16).  Short K stays on 64x64 BK 32, which has the
    // persistent kernel, and so does N <= 64 (C5 P.V: 170.3 us against 174.0).
    if (!gathered && tiles(kTileM) > 3 * cus && k > 256 && n > 64) return kTileH;
    return kTileM;
}

// Split-K factor.  A problem of at least half a workgroup per CU takes the
// split S that minimises its makespan, ceil(T*S/CUs) workgroups on the
// busiest CU each running K/S: min over S of ceil(T*S/CUs) / S (a larger S
// must gain at least 5%, which the reduce pass costs: 3000^3 TN is 446 us
// unsplit against 467 us in 3 for a 3.7% smaller makespan), with at
// least 768 of K per slice (below that the reduce costs more than it saves:
// 1000^3 26.0 us unsplit, 30.3 us in 2) and at most 16 slices.  On a tie the
// smaller S wins, except that an S giving two or more workgroups per CU beats
// one that leaves a single workgroup (4 waves) per CU (1024x1024x4096 TN:
// 84.7 us unsplit, 78 us in 2-4).  Measured on MI355X: 1000x600x3000 TN
// 59 -> 44 us (2 -> 3 slices), 1536^3 NN 81.6 -> 74.3 us (1 -> 3),
// 4097^2 x 4096 NN 1495 -> 1256 us (1 -> 3), 1280^2 x 2560 NN 91.8 -> 83.6 us
// (1 -> 3).  The partial sums may take at most 256 MiB of workspace.
// Fewer tiles than half the CUs: aim at 2*CUs workgroups with >= 128 of K
// per slice (>= 64 when there are at most 8 tiles), at most 16 slices, 64
// when K >= 16384 (long reductions such as a conv weight gradient over a
// whole batch).
int choose_splits(const zn_ctx *ctx, Tile tile, int64_t m, int64_t n, int64_t k, int64_t batch) {
    const int64_t cus = cus_now(ctx);
    const TileShape &ts = kTiles[tile];
    const int64_t tiles = cdiv(m, ts.bm) * cdiv(n, ts.bn) * batch;
    // The 128x128 BK 32 tile runs one workgroup per CU: a second workgroup
    // per CU is a second round (2048x2048x1536 NN 119.9 us in 2 slices
    // against 106.8 us unsplit), so its split only fills the first.
    if (tile == kTileR) return (int)round_splits(tiles, k, cus);
    if (tiles >= cus / 2) {
        int64_t best = 1, best_load = cdiv(tiles, cus);  // workgroups on the busiest CU
        const int64_t max_s = std::min<int64_t>(16, k / 768);
        constexpr int64_t kMaxWorkspaceFloats = (int64_t)1 << 26;  // 256 MiB of partial sums
        for (int64_t sp = 2; sp <= max_s && sp * batch * m * n <= kMaxWorkspaceFloats; ++sp) {
            const int64_t load = cdiv(tiles * sp, cus);
            // load / sp at least 5% below best_load / best (the reduce pass costs a few percent)
            const bool faster = load * best * 20 < best_load * sp * 19;
            const bool tie_more_waves = load * best == best_load * sp && best_load < 2 && load >= 2;
            if (faster || tie_more_waves) {
                best = sp;
                best_load = load;
            }
        }
        return (int)best;
    }
    int64_t splits = std::min<int64_t>(2 * cus / tiles, k / (tiles <= 8 ? 64 : 128));
    const int64_t cap = k >= 16384 ? 64 : 16;
    if (splits > cap) splits = cap;
    return splits < 2 ? 1 : (int)splits;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Multiplier and shift for x / d, 0 <= x < 2^31, d >= 1: shift = ceil(log2 d),
// mul = ceil(2^(31 + shift) / d), which is below 2^32 (Granlund & Montgomery
// 1994, Theorem 4.2 with N = 31).
void udiv_magic(uint32_t d, uint32_t &mul, uint32_t &shift) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    mul = (uint32_t)(((1ull << (31 + l)) + d - 1) / d);
    shift = l;
}

// Gathered B operands (ZnConvGeom), selected by `conv` + `mode`:
//  kGatherIm2col:     the implicit im2col operand of an NCHW image batch
//                     (images `stride_b` apart), NN with M = out channels,
//                     N = out pixels;
//  kGatherTransposed: the transposed-convolution operand of a stride-1 input
//                     gradient (B[n][k] from [OH*OW][OC] grad_output rows,
//                     K-contiguous 16-byte chunks), NT with M = in channels,
//                     N = in pixels;
//  kGatherWeightGrad: the col operand of a weight gradient (B[k][n] =
//                     col[pixel][tap] over conv->images images, K-contiguous
//                     4-pixel chunks), TN with M = out channels, N = taps;
//  kGatherNhwc:       the implicit im2col operand of an NHWC image batch
//                     (B[n][k], K-contiguous 4-channel chunks), NT with
//                     M = out channels, N = out pixels;
//  kGatherWeightNhwc: the col operand of a weight gradient from an NHWC
//                     batch (B[k][n], X-contiguous 4-channel chunks), TN like
//                     kGatherWeightGrad.
enum GatherMode { kGatherIm2col, kGatherTransposed, kGatherWeightGrad, kGatherNhwc, kGatherWeightNhwc };

constexpr double kPackMinMacs = 536870912.0;  // 2^29 multiply-adds: the copy costs a few us

// Rows of C after the m rows of a launch that the launch may compute as
// well (folded row tail): A's first tail row (TN: column), C's first tail
// row, their count.  `folded` reports whether it did.
struct RowTail {
    const float *a;
    float *c;
    int64_t rows;
    bool folded;
};

// split_rows: the launch may cut itself into two launches (a row tail; the
// last problems of a batch), whose calls pass false.
int gemm_launch_ex(zn_ctx *ctx, int layout, int64_t m, int64_t n, int64_t k, const float *a, int64_t lda,
                   int64_t stride_a, const float *b, int64_t ldb, int64_t stride_b, float *c, int64_t ldc,
                   int64_t stride_c, int64_t batch, int accumulate, const float *bias, int act, int bias_rows,
                   const ZnConvGeom *conv = nullptr, GatherMode mode = kGatherIm2col, bool split_rows = true,
                   int padded = 0, RowTail *row_tail = nullptr) {
    if (!ctx) return ZN_ERR_INVALID_ARG;
    if (layout < ZN_LAYOUT_NN || layout > ZN_LAYOUT_TN) return ZN_ERR_INVALID_ARG;
    if (act < ZN_ACT_LINEAR || act > ZN_ACT_TANH) return ZN_ERR_INVALID_ARG;
    if (m < 0 || n < 0 || k < 0 || batch < 0 || stride_a < 0 || stride_b < 0 || stride_c < 0)
        return ZN_ERR_INVALID_ARG;
    if (m > INT_MAX || n > INT_MAX || k > INT_MAX) return ZN_ERR_OVERFLOW;
    if (m == 0 || n == 0 || batch == 0) return ZN_OK;
    if (!c || (k > 0 && (!a || !b))) return ZN_ERR_INVALID_ARG;
    // stored row lengths: A is [m x k] (nn, nt) or [k x m] (tn); B is [k x n] (nn, tn) or [n x k] (nt)
    const int64_t a_row = layout == ZN_LAYOUT_TN ? m : k;
    const int64_t b_row = layout == ZN_LAYOUT_NT ? k : n;
    if (k > 0 && (lda < a_row || ldb < b_row || lda < 1 || ldb < 1)) return ZN_ERR_INVALID_ARG;
    if (ldc < n) return ZN_ERR_INVALID_ARG;
    // The kernels address each operand of one problem with 32-bit byte
    // offsets: keep every per-problem extent below 2 GiB.
    const int64_t a_outer = layout == ZN_LAYOUT_TN ? k : m;
    const int64_t b_outer = layout == ZN_LAYOUT_NT ? n : k;
    const int64_t kLimit = (int64_t)INT_MAX / 4;
    const bool weight_mode = mode == kGatherWeightGrad || mode == kGatherWeightNhwc;
    const int64_t images = conv && weight_mode ? conv->images : 1;
    const int64_t b_extent =
        conv ? images * conv->channels * conv->in_h * conv->in_w : (b_outer - 1) * ldb + b_row;
    if (k > 0 && ((a_outer - 1) * lda + a_row > kLimit || b_extent > kLimit)) return ZN_ERR_OVERFLOW;
    constexpr int kGatherLayout[5] = {ZN_LAYOUT_NN, ZN_LAYOUT_NT, ZN_LAYOUT_TN, ZN_LAYOUT_NT, ZN_LAYOUT_TN};
    if (conv && layout != kGatherLayout[mode]) return ZN_ERR_INVALID_ARG;
    if (conv && (mode == kGatherTransposed || mode == kGatherNhwc) &&
        (k % 4 != 0 || conv->channels % 4 != 0 || !aligned16(b) || stride_b % 4 != 0))
        return ZN_ERR_INVALID_ARG;  // whole 16-byte chunks of 4 channels
    if (conv && mode == kGatherWeightGrad &&
        (conv->stride_w != 1 || conv->out_w % 4 != 0 || conv->k_order != 0 || batch != 1 ||
         k != images * conv->out_h * conv->out_w))
        return ZN_ERR_INVALID_ARG;  // whole 4-pixel chunks of one output row, over all images
    if (conv && mode == kGatherWeightNhwc &&
        (conv->channels % 4 != 0 || conv->k_order != 0 || batch != 1 || !aligned16(b) ||
         k != images * conv->out_h * conv->out_w))
        return ZN_ERR_INVALID_ARG;  // whole 4-channel chunks, over all images

    // The NHWC forward gather runs best on 64x64 tiles (C5 forward, rocprofv3 trace: 156 us against 172 us for
    // 128x128 and 314 us for 256x128).
    // A forced tile without convolution kernels leaves convolutions to the policy.
    const bool forced = ctx->forced_tile >= 0 && (!conv || kTiles[ctx->forced_tile].conv);
    // 16-byte staging of both operands as they lie (the tiles without a
    // 4-byte kernel need it; packed copies are not made for them)
    const bool native_vec = !conv && aligned16(a) && aligned16(b) && lda % 4 == 0 && ldb % 4 == 0 && stride_a % 4 == 0 &&
                            stride_b % 4 == 0 && a_row % 4 == 0 && b_row % 4 == 0;
    // The NHWC weight gradient (a long K over every output pixel, few tiles)
    // runs as one round of 128x128 tiles x K slices on the register-staged
    // loop when grad_output's rows are whole float4s: up to 64 slices, one
    // workgroup per CU (MI355X, C5 128 x 576 x 100352: the GEMM 175 -> 155
    // us against 64x64 tiles in 64 slices, the whole backward 334 -> 323 us).
    const bool wn_wide = conv && mode == kGatherWeightNhwc && aligned16(a) && lda % 4 == 0 && stride_a % 4 == 0 &&
                         a_row % 4 == 0 && cdiv(m, 128) * cdiv(n, 128) * 2 <= cus_now(ctx) && k >= 64 * 128;
    Tile tile = forced                        ? (Tile)ctx->forced_tile
                : conv && mode == kGatherNhwc ? kTileM
                : wn_wide                     ? kTileR
                                              : choose_tile(ctx, m, n, k, batch, conv != nullptr, native_vec);
    if (!kTiles[tile].plain && !native_vec) tile = kTileX;  // forced onto a tile it cannot stage: 256x128
    const TileShape &ts = kTiles[tile];
    const int64_t tiles_m = cdiv(m, ts.bm), tiles_n = cdiv(n, ts.bn);
    if (tiles_m * tiles_n > INT_MAX) return ZN_ERR_OVERFLOW;

    // Row tail: when the last row of tiles is what puts one more workgroup on
    // the busiest CU (1040 tiles of 64x64 for 4097 x 1023: 5 on some CUs, 4
    // on the rest), the rows above it run as one GEMM and the tail rows as a
    // second, small one (usually the intra-workgroup split-K kernel).  Each
    // part is an ordinary GEMM of its rows, so no element changes its K order
    // in the first part.  Each part then makes its own staging choices.
    if (split_rows && !conv && batch == 1 && k > 0 && ctx->forced_tile < 0 && ctx->forced_splits == 0 &&
        ctx->forced_wave_split < 0 && tiles_m >= 2) {
        const int64_t cus = cus_now(ctx);
        const int64_t ntiles_all = tiles_m * tiles_n;
        const int64_t per_cu = cdiv(ntiles_all, cus);
        if (per_cu >= 2 && cdiv(ntiles_all - tiles_n, cus) < per_cu) {
            const int64_t m_main = (tiles_m - 1) * ts.bm;
            const float *a_tail = layout == ZN_LAYOUT_TN ? a + m_main : a + m_main * lda;
            // the first part may compute the tail rows too (below); if not, they are a second launch
            RowTail tail = {a_tail, c + m_main * ldc, m - m_main, false};
            int rc = gemm_launch_ex(ctx, layout, m_main, n, k, a, lda, 0, b, ldb, 0, c, ldc, 0, 1, accumulate, bias,
                                    act, bias_rows, nullptr, mode, false, padded, &tail);
            if (rc || tail.folded) return rc;
            return gemm_launch_ex(ctx, layout, m - m_main, n, k, a_tail, lda, 0, b, ldb, 0, c + m_main * ldc, ldc, 0, 1,
                                  accumulate, bias_rows ? bias + m_main : bias, act, bias_rows, nullptr, mode, false,
                                  padded);
        }
    }
    // The 128x128 register-staged tile loads rows that are not whole float4s
    // as they lie, 16 bytes at a time (the _u kernels), unless the problem
    // takes the intra-workgroup split-K kernels below: no packed copies, no
    // 4-byte staging.
    const bool wave_split_possible =
        !conv && k > 0 &&
        (ctx->forced_wave_split > 0 ||
         (ctx->forced_wave_split < 0 && ctx->forced_tile < 0 && ctx->forced_splits == 0 &&
          cdiv(m, 32) * cdiv(n, 32) * batch <= cus_now(ctx) && k >= 64 && k <= 4096));
    const bool unaligned = !conv && tile == kTileR && !native_vec && k > 0 && !wave_split_possible;

    // Operands whose rows are not 16-byte aligned whole float4s would be
    // staged with 4-byte loads (4x the load instructions).  For large single
    // problems they are first copied into zero-padded aligned rows (C4
    // 4097x1023x777: 95 us with 4-byte staging, the GEMM alone 75 us with
    // 16-byte staging); the padding adds exact zeros past K, which the 4-byte
    // path stages as well, so the result is the same.
    Lease pack_a(ctx), pack_b(ctx);
    // rows padded with zeros to whole float4s (here, or by the caller: padded bit 0 = A, bit 1 = B)
    bool a_packed = (padded & 1) != 0, b_packed = (padded & 2) != 0;
    if (!conv && !unaligned && !ctx->no_alloc && batch == 1 && k > 0 && (double)m * n * k >= kPackMinMacs) {
        const bool a_vec = aligned16(a) && lda % 4 == 0 && a_row % 4 == 0;
        const bool b_vec = aligned16(b) && ldb % 4 == 0 && b_row % 4 == 0;
        // both packings go into one launch (blockIdx.y selects the operand)
        ZnPack2Args jobs;
        std::memset(&jobs, 0, sizeof(jobs));
        int njobs = 0;
        int64_t most = 0;  // float4s of the larger packed operand
        auto pack = [&](Lease &l, const float *&src, int64_t &ld, int64_t rows, int64_t cols, bool &packed) -> int {
            const int64_t ld_dst = (cols + 3) & ~(int64_t)3;
            if ((rows - 1) * ld_dst + ld_dst > kLimit) return ZN_OK;  // stays on the 4-byte path
            int rc2 = l.get((size_t)(rows * ld_dst));
            if (rc2) return rc2;
            ZnPackArgs &pa = jobs.op[njobs++];
            pa.src = src;
            pa.dst = l.ptr;
            pa.rows = rows;
            pa.cols = cols;
            pa.ld_src = ld;
            pa.ld_dst = ld_dst;
            most = std::max<int64_t>(most, rows * ld_dst / 4);
            src = l.ptr;
            ld = ld_dst;
            packed = true;
            return ZN_OK;
        };
        int rcp;
        if (!a_vec && !a_packed && (rcp = pack(pack_a, a, lda, a_outer, a_row, a_packed))) return rcp;
        if (!b_vec && !b_packed && (rcp = pack(pack_b, b, ldb, b_outer, b_row, b_packed))) return rcp;
        if (njobs > 0) {
            const int64_t cap = cus_now(ctx) * 16;
            if ((rcp = select_device(ctx)) ||
                (rcp = launch(ctx, ctx->elt[kPack], (unsigned)std::min<int64_t>(cdiv(most, 256), cap), (unsigned)njobs,
                              256, &jobs)))
                return rcp;
        }
    }

    ZnGemmArgs args;
    std::memset(&args, 0, sizeof(args));
    args.a = a;
    args.b = b;
    args.c = c;
    args.bias = bias;
    args.lda = lda;
    args.ldb = ldb;
    args.ldc = ldc;
    args.stride_a = stride_a;
    args.stride_b = stride_b;
    args.stride_c = stride_c;
    args.m = (int32_t)m;
    args.n = (int32_t)n;
    args.k = (int32_t)k;
    args.tiles_m = (int32_t)tiles_m;
    args.tiles_n = (int32_t)tiles_n;
    args.accumulate = accumulate ? 1 : 0;
    args.act = act;
    args.bias_rows = bias_rows ? 1 : 0;
    if (conv) args.conv = *conv;
    // NHWC forward: each BK slice of K lies in one filter tap when the channels are whole slices
    if (conv && mode == kGatherNhwc) args.conv.tap_uniform = conv->channels % ts.bk == 0 ? 1 : 0;
    // 16-byte staging: aligned rows and contiguous extents that are whole float4s
    const bool vec = conv ? (aligned16(a) && lda % 4 == 0 && stride_a % 4 == 0 && a_row % 4 == 0)
                          : (aligned16(a) && aligned16(b) && lda % 4 == 0 && ldb % 4 == 0 && stride_a % 4 == 0 &&
                             stride_b % 4 == 0 && (a_row % 4 == 0 || a_packed) && (b_row % 4 == 0 || b_packed));
    args.vec_c = aligned16(c) && ldc % 4 == 0 && stride_c % 4 == 0;
    // Plain row-major tile order: on MI355X it gave the lowest L2-miss traffic
    // for multi-round problems (8192^3 NN: 5.6 GB fetched per launch against
    // 6.2-28 GB for 2-32-row groups and XCD-contiguous remapping), at equal
    // speed; single-round problems are indifferent.
    args.group_m = 1;
    const int64_t ntiles = tiles_m * tiles_n;
    args.xcd_remap = 0;

    // Batched transposed-convolution GEMMs (the convolution input gradient,
    // one problem per image) whose tiles overrun the resident workgroups by
    // a short last round: those few tiles would run nearly alone at the end
    // (MI355X, C5's 49 tiles per image on 1536 resident workgroups: 147.8 us
    // for 31 images, 168.8 us for 32).  The last problems go to a launch of
    // their own, which the split-K policy spreads over every CU.
    if (conv && mode == kGatherTransposed && split_rows && batch > 1 && !forced && ctx->forced_splits == 0) {
        const int64_t slots = cus_now(ctx) * ctx->convt_occ[tile][vec ? 1 : 0];
        const int64_t total = ntiles * batch, rem = total % slots;
        const int64_t r = cdiv(rem, ntiles);  // problems holding the last round's tiles
        if (total > slots && rem > 0 && 8 * rem <= slots && r < batch) {
            const int64_t b1 = batch - r;
            const int rc = gemm_launch_ex(ctx, layout, m, n, k, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c, b1,
                                          accumulate, bias, act, bias_rows, conv, mode, false, padded);
            if (rc) return rc;
            return gemm_launch_ex(ctx, layout, m, n, k, a + b1 * stride_a, lda, stride_a, b + b1 * stride_b, ldb,
                                  stride_b, c + b1 * stride_c, ldc, stride_c, r, accumulate, bias, act, bias_rows, conv,
                                  mode, false, padded);
        }
    }

    int rc = select_device(ctx);
    if (rc) return rc;
    constexpr int64_t kMaxGridY = 65535;
    const int64_t chunk_batch = batch < kMaxGridY ? batch : kMaxGridY;
    int splits;
    if (ctx->forced_splits > 0) {
        splits = (int)std::min<int64_t>(ctx->forced_splits, std::max<int64_t>(1, cdiv(k, ts.bk)));
    } else if (wn_wide && !forced) {  // one round: CUs / tiles slices, at most 64, at least 768 of K each
        const int64_t wn_tiles = cdiv(m, 128) * cdiv(n, 128);
        splits = (int)std::max<int64_t>(1, std::min<int64_t>({64, cus_now(ctx) / wn_tiles, k / 768}));
    } else {
        splits = choose_splits(ctx, tile, m, n, k, batch);
    }
    int64_t k_chunk = k;
    if (splits > 1) {
        k_chunk = cdiv(cdiv(k, splits), ts.bk) * ts.bk;
        splits = (int)cdiv(k, k_chunk);
        const size_t need = (size_t)splits * (size_t)chunk_batch * (size_t)m * (size_t)n * sizeof(float);
        if (ctx->no_alloc) {
            // partial sums in the fixed scratch: a split the caller forced
            // must fit it; the policy's own split falls back to one pass
            if (need > kScratchBytes) {
                if (ctx->forced_splits > 0) return ZN_ERR_INVALID_ARG;
                splits = 1;
            }
        } else if (splits > 1 && ensure_workspace(ctx, need) != ZN_OK) {
            splits = 1;  // fall back to one pass
        }
        if (splits <= 1) {
            splits = 1;
            k_chunk = k;
        }
    }
    args.splits = splits;
    args.k_chunk = (int32_t)k_chunk;
    float *const ws = ctx->no_alloc ? ctx->scratch : ctx->ws;
    args.ws = ws;
    // 4-pixel (16-byte) gather: unit column stride, and whole chunks of 4 pixels per output row
    const int gather4 = conv && conv->stride_w == 1 && conv->out_w % 4 == 0 ? 1 : 0;
    const int staging = unaligned ? 2 : vec ? 1 : 0;  // 4-byte, 16-byte, 16-byte unaligned
    hipFunction_t f = !conv                     ? ctx->gemm[layout][tile][staging]
                      : mode == kGatherTransposed ? ctx->convt[tile][vec ? 1 : 0]
                      : mode == kGatherWeightGrad ? ctx->convw[tile][vec ? 1 : 0]
                      : mode == kGatherNhwc       ? ctx->convf[tile][vec ? 1 : 0]
                      : mode == kGatherWeightNhwc ? ctx->convwn[tile][vec ? 1 : 0]
                                                  : ctx->conv[tile][vec ? 1 : 0][gather4];
    // Problems of at most one 32x32 tile per CU: one launch in which the
    // waves of each workgroup split K among themselves and sum their partial
    // tiles in LDS in wave order (gemm_ksplit), instead of split-K slices in
    // separate workgroups plus a reduce launch.  On MI355X: C1 512^3 12.6 ->
    // 6.3 us, the C2 GEMMs 7.7-12.2 -> 4.1-9.3 us; with 1024 tiles (1000^3)
    // or more the tiled kernels win.  Four waves below K = 512, eight above.
    // Tiles for at most half the CUs with K >= 1536 also split K over up to
    // cus / tiles workgroups of four waves (at most 32 slices of 32 or more),
    // whose partial tiles the last workgroup of each tile adds in slice order
    // in the same launch.  On MI355X: 300 x 200 x 3000 27.4 -> 20.1 us; the
    // hand-over (stores, counter, the last workgroup's loads) costs about
    // 5 us, so below K = 1536 (C2's 256 x 128 x 784: 9.7 us unsplit, 14.1
    // split 7 ways) one workgroup per tile stays faster.
    {
        const int64_t cus = cus_now(ctx);
        const int64_t tiles32 = cdiv(m, 32) * cdiv(n, 32) * batch;
        int waves = 0;
        if (!conv && k > 0 && ctx->forced_wave_split > 0)
            waves = ctx->forced_wave_split;
        else if (!conv && ctx->forced_wave_split < 0 && ctx->forced_tile < 0 && ctx->forced_splits == 0 &&
                 tiles32 <= cus && k >= 64 && k <= 4096)
            waves = k >= 512 ? 8 : 4;
        // 16x16 tiles (four waves splitting K) for at most one round of them,
        // unless they are so few that the workgroup split below does better
        // (K >= 1536 and 16x16 tiles for under half the CUs).  On MI355X:
        // C2's 256 x 128 x 784 forward 9.1 -> 5.6 us, 256 x 10 x 128
        // 5.8 -> 4.0 us, 300 x 200 x 3000 15.3 us (18.7 split over
        // workgroups); 64 x 64 x 4096 17.7 us against 14.1 split.  Up to
        // three per CU run on the two-stage kernels (several workgroups per
        // CU): 384^3 5.7 -> 4.9 us, 512 x 256 x 1024 9.5 -> 6.5 us; C1's
        // 512^3 (four per CU) stays on 32x32 tiles (6.2 against 6.4 us).
        const int64_t tiles16 = cdiv(m, 16) * cdiv(n, 16) * batch;
        if (waves == 16 || (waves && ctx->forced_wave_split < 0 &&
                            ((tiles16 <= cus && (k < 1536 || tiles16 * 2 >= cus)) ||
                             (tiles16 > cus && tiles16 <= 3 * cus)))) {
            ZnGemmArgs q = args;
            q.tiles_m = (int32_t)cdiv(m, 16);
            q.tiles_n = (int32_t)cdiv(n, 16);
            q.splits = 1;
            q.k_chunk = (int32_t)k;
            if ((int64_t)q.tiles_m * q.tiles_n > INT_MAX) return ZN_ERR_OVERFLOW;
            for (int64_t b0 = 0; b0 < batch; b0 += kMaxGridY) {
                const int64_t nb = batch - b0 < kMaxGridY ? batch - b0 : kMaxGridY;
                ZnGemmArgs part = q;
                part.batch = (int32_t)nb;
                part.a = a + b0 * stride_a;
                part.b = b + b0 * stride_b;
                part.c = c + b0 * stride_c;
                // one workgroup per CU at most: eight waves of one stage each
                // once K holds 8 slices or more (C2's 256 x 128 x 784 5.5 ->
                // 4.65 us, 300 x 200 x 3000 15.3 -> 11.7 us), else four waves
                // with every slice in flight (256 x 10 x 128: 3.3 against 3.9 us)
                const int qr = tiles16 > cus ? 1 : k >= 8 * 32 ? 2 : 0, qv = vec ? 1 : 0;
                rc = launch(ctx, ctx->gemmq[layout][qr][qv], (unsigned)(q.tiles_m * q.tiles_n), (unsigned)nb,
                            (unsigned)ctx->gemmq_threads[layout][qr][qv], &part);
                if (rc) return rc;
            }
            return ZN_OK;
        }
        if (waves) {
            ZnGemmArgs kargs = args;
            kargs.tiles_m = (int32_t)cdiv(m, 32);
            kargs.tiles_n = (int32_t)cdiv(n, 32);
            kargs.splits = 1;
            kargs.k_chunk = (int32_t)k;
            // K in slices of `chunk` (a multiple of 32), slice q to wave q % 4
            // of workgroup q / 4: the slices of the 32x32 tile split into as
            // many parts by the split-K launches, added in the same order
            int64_t wsplits = 1;
            if (ctx->forced_wave_split < 0 && tiles32 * 2 <= cus && tiles32 <= kCounterSlots && k >= 1536)
                wsplits = std::min<int64_t>({cus / tiles32, cdiv(k, 4 * 32), 8});
            if (wsplits >= 2) {
                const int64_t chunk = cdiv(cdiv(k, 4 * wsplits), 32) * 32;
                wsplits = cdiv(cdiv(k, chunk), 4);
                const size_t need = (size_t)(tiles32 * wsplits) * 4 * 32 * 32 * sizeof(float);
                if (ctx->no_alloc ? need > kScratchBytes : ensure_workspace(ctx, need) != ZN_OK) wsplits = 1;
                if (wsplits >= 2) {
                    waves = 4;
                    kargs.splits = (int32_t)wsplits;
                    kargs.k_chunk = (int32_t)chunk;
                    kargs.ws = ctx->no_alloc ? ctx->scratch : ctx->ws;
                    kargs.counters = ctx->counters;
                }
            }
            hipFunction_t fk = kargs.splits > 1 ? ctx->gemmks[layout][vec ? 1 : 0]
                                                : ctx->gemmk[layout][waves == 8 ? 1 : 0][vec ? 1 : 0];
            for (int64_t b0 = 0; b0 < batch; b0 += kMaxGridY) {
                const int64_t nb = batch - b0 < kMaxGridY ? batch - b0 : kMaxGridY;
                ZnGemmArgs part = kargs;
                part.batch = (int32_t)nb;
                part.a = a + b0 * stride_a;
                part.b = b + b0 * stride_b;
                part.c = c + b0 * stride_c;
                rc = launch(ctx, fk, (unsigned)(kargs.tiles_m * kargs.tiles_n), (unsigned)nb, (unsigned)(waves * 64),
                            &part, (unsigned)kargs.splits);
                if (rc) return rc;
            }
            return ZN_OK;
        }
    }
    // Plain unsplit GEMMs with short K (at most 8 slices per tile) and more
    // than one round of tiles run on the persistent kernels: as many
    // workgroups as can be resident, each walking its share of the (problem,
    // tile) items with the LDS pipeline running on across tiles, so no tile
    // waits for a fresh dispatch and its first load (C5 QK^T, K = 64:
    // 232 -> 215 us).  Longer tiles keep the hardware's dynamic assignment,
    // which balances the CUs better (C5 convolution GEMM, K = 576: 132 us
    // plain, 150 us persistent; 8192^3 0.6% slower persistent).
    if (!conv && splits == 1 && vec && k > 0 && kTiles[tile].persistent && ctx->forced_persistent != 0) {
        const int64_t cus = cus_now(ctx);
        const int64_t total = ntiles * batch;
        ZnGemmArgs part = args;
        part.batch = (int32_t)batch;
        // Deferred stores (gemm_persistent_defer) for plain problems whose
        // 128x128 tiles all lie inside C, K of 4 slices or more, and more
        // tiles than its own resident workgroups (two per CU): C5 QK^T
        // 203 -> 184 us, 4096^2 x 64 NN 33.5 -> 26.4 us (plain kernels: its
        // 1024 tiles fit the plain persistent kernel's residency), 1024^2 x
        // 80 TN x 32 68.0 -> 53.9 us, 1024^2 x 128 NT x 64 164.9 -> 157.0 us.
        const bool defer_ok = ctx->forced_persistent != 1 && tile == kTileL && !accumulate && !bias &&
                              act == ZN_ACT_LINEAR && m % 128 == 0 && n % 128 == 0 && k > 48 &&
                              (layout == ZN_LAYOUT_NT || args.vec_c) && total <= INT_MAX;
        const int64_t resident_d = cus * (int64_t)ctx->gemmpd_occ[layout];
        if (defer_ok && (ctx->forced_persistent == 2 || (total > resident_d && k <= 8 * (int64_t)ts.bk))) {
            const int64_t grid = std::min(total, resident_d);
            // each XCD walks a contiguous run of items: C5 QK^T fetched 302 MB
            // per launch, 68 MB with the remap (Q and K are 64 MB), 2% faster
            if (grid >= 8) part.xcd_remap = 3;
            hipFunction_t fd = cdiv(k, 16) == 4 ? ctx->gemmpd4[layout] : ctx->gemmpd[layout];
            return launch(ctx, fd, (unsigned)grid, 1, (unsigned)ctx->gemmpd_threads[layout], &part);
        }
        const int64_t resident = cus * ctx->gemmp_occ[layout][tile];
        if (total <= INT_MAX &&
            (ctx->forced_persistent >= 1 || (total > resident && k <= 8 * (int64_t)ts.bk)))
            return launch(ctx, ctx->gemmp[layout][tile], (unsigned)std::min(total, resident), 1,
                          (unsigned)ts.threads, &part);
    }
    for (int64_t b0 = 0; b0 < batch; b0 += kMaxGridY) {
        const int64_t nb = batch - b0 < kMaxGridY ? batch - b0 : kMaxGridY;
        ZnGemmArgs part = args;
        part.batch = (int32_t)nb;
        if (splits > 1 && nb == 1) part.xcd_remap = 2;  // the tiles of one K slice share an XCD's L2
        part.a = a ? a + b0 * stride_a : nullptr;
        part.b = b ? b + b0 * stride_b : nullptr;
        part.c = c + b0 * stride_c;
        // A few tail rows go with the unaligned 128x128 tiles when each
        // workgroup gets at most 4 of their elements and K <= 1024 (two
        // products per thread): each element a dot product spread over one
        // workgroup's 512 threads, whose operands load before the main loop.
        // C4 4097 x 1023 x 777: the one-row tail needs no second launch.
        if (row_tail && unaligned && batch == 1 && k <= 1024) {
            const int64_t wgs = ntiles * splits;
            const int64_t per = cdiv(row_tail->rows * n, wgs);
            if (per <= 4 && row_tail->rows * n <= INT_MAX) {
                part.tail_a = row_tail->a;
                part.tail_c = row_tail->c;
                part.tail_rows = (int32_t)row_tail->rows;
                part.tail_per_wg = (int32_t)per;
                row_tail->folded = true;
            }
        }
        const int threads = conv ? ts.threads : ctx->gemm_threads[layout][tile][staging];
        rc = launch(ctx, f, (unsigned)ntiles, (unsigned)nb, (unsigned)threads, &part, (unsigned)splits);
        if (rc) return rc;
        if (splits > 1) {
            ZnReduceArgs r;
            std::memset(&r, 0, sizeof(r));
            r.ws = ws;
            r.c = part.c;
            r.bias = bias;
            r.ldc = ldc;
            r.stride_c = stride_c;
            r.m = (int32_t)m;
            r.n = (int32_t)n;
            r.batch = (int32_t)nb;
            r.splits = splits;
            r.accumulate = accumulate ? 1 : 0;
            r.act = act;
            r.bias_rows = bias_rows ? 1 : 0;
            r.vec = (n % 4 == 0 && ldc % 4 == 0 && stride_c % 4 == 0 && aligned16(part.c)) ? 1 : 0;
            const int64_t items = m * n * nb / (r.vec ? 4 : 1);
            int64_t blocks = cdiv(items, 256);
            const int64_t cap = cus_now(ctx) * 8;
            if (blocks > cap) blocks = cap;
            rc = launch(ctx, ctx->splitk_reduce, (unsigned)blocks, 1, 256, &r);
            if (rc) return rc;
        }
    }
    return ZN_OK;
}

int gemm_launch(zn_ctx *ctx, int layout, int64_t m, int64_t n, int64_t k, const float *a, int64_t lda,
                int64_t stride_a, const float *b, int64_t ldb, int64_t stride_b, float *c, int64_t ldc,
                int64_t stride_c, int64_t batch, int accumulate, const float *bias, int act) {
    return gemm_launch_ex(ctx, layout, m, n, k, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c, batch,
                          accumulate, bias, act, 0);
}

template <typename Args>
int elt_launch(zn_ctx *ctx, EltKernel kernel, int64_t work_items, const Args &args) {
    int rc = select_device(ctx);
    if (rc) return rc;
    const int64_t threads = 256;
    int64_t blocks = cdiv(work_items, threads);
    const int64_t cap = cus_now(ctx) * 16;
    if (blocks > cap) blocks = cap;  // grid-stride loops cover the rest
    if (blocks < 1) blocks = 1;
    Args a = args;
    return launch(ctx, ctx->elt[kernel], (unsigned)blocks, 1, (unsigned)threads, &a);
}

constexpr size_t kStageBytes = (size_t)32 << 20;  // per pinned staging buffer
constexpr size_t kStageMin = (size_t)4 << 20;      // smaller copies stay pageable

// Set-up fault injection for the error-path tests: with
// ZN_HIP_ENABLE_TEST_HOOKS=1, ZN_HIP_TEST_SETUP_FAULT=n makes step n of the
// staging (1-5) or pipeline (11-21) set-up fail as if the HIP call had run
// out of memory.  Both are read at each set-up attempt; without the first
// the second is ignored, so a stray variable cannot fail a production call.
hipError_t setup_step(int step, hipError_t real) {
    const char *on = std::getenv("ZN_HIP_ENABLE_TEST_HOOKS");
    if (!on || std::strcmp(on, "1") != 0) return real;
    const char *env = std::getenv("ZN_HIP_TEST_SETUP_FAULT");
    if (env && std::atoi(env) == step) return hipErrorOutOfMemory;
    return real;
}

void release_staging(zn_ctx *ctx) {
    ctx->copier.reset();
    for (int i = 0; i < 2; ++i) {
        if (ctx->pinned_done[i]) (void)hipEventDestroy(ctx->pinned_done[i]);
        if (ctx->pinned[i]) (void)hipHostFree(ctx->pinned[i]);
        ctx->pinned_done[i] = nullptr;
        ctx->pinned[i] = nullptr;
    }
}

// The staging set is ready only when complete (the copier is made last); a
// failed set-up releases what it made, so a later call starts afresh.
int ensure_staging(zn_ctx *ctx) {
    if (ctx->copier) return ZN_OK;
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        e = setup_step(1 + 2 * i, hipHostMalloc((void **)&ctx->pinned[i], kStageBytes, hipHostMallocDefault));
        if (e == hipSuccess)
            e = setup_step(2 + 2 * i, hipEventCreateWithFlags(&ctx->pinned_done[i], hipEventDisableTiming));
    }
    if (e == hipSuccess) e = setup_step(5, hipSuccess);
    if (e != hipSuccess) {
        release_staging(ctx);
        return fail_hip(ctx, e, e == hipErrorOutOfMemory ? ZN_ERR_OOM : ZN_ERR_HIP);
    }
    const unsigned hw = std::thread::hardware_concurrency();
    ctx->copier.reset(new HostCopier((int)std::min(15u, hw > 1 ? hw - 1 : 0u)));
    return ZN_OK;
}

// Work queued on a stream that reads or writes pinned staging memory must be
// finished before that memory is used again, also when the call returns
// early with an error.  Declared after the call's leases, so it waits before
// they go back to the pool.
struct PinnedFence {
    zn_ctx *ctx;
    hipStream_t stream = nullptr;  // the context stream when null
    bool done = false;
    ~PinnedFence() {
        if (!done) (void)hipStreamSynchronize(stream ? stream : ctx->stream);
    }
};

// Host -> device on `stream` (the context stream by default).  Large copies:
// chunk i is copied into pinned buffer i % 2 once that buffer's previous DMA
// has finished, then DMAed; host copies and DMAs of consecutive chunks
// overlap.  Host-slice calls are not capturable (they read and write host
// memory synchronously).
int copy_in(zn_ctx *ctx, float *dst, const float *src, size_t n, hipStream_t stream = nullptr) {
    if (ctx->capturing) return ZN_ERR_INVALID_ARG;
    if (n == 0) return ZN_OK;
    if (!stream) stream = ctx->stream;
    const size_t bytes = n * sizeof(float);
    if (bytes < kStageMin) {
        ZN_HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream));
        return ZN_OK;
    }
    int rc = ensure_staging(ctx);
    if (rc) return rc;
    PinnedFence fence{ctx, stream};
    for (size_t off = 0, i = 0; off < bytes; off += kStageBytes, ++i) {
        const size_t len = std::min(kStageBytes, bytes - off);
        const int s = (int)(i & 1);
        ZN_HIP_TRY(ctx, hipEventSynchronize(ctx->pinned_done[s]));  // its previous DMA has read it
        ctx->copier->copy(ctx->pinned[s], (const char *)src + off, len);
        ZN_HIP_TRY(ctx, hipMemcpyAsync((char *)dst + off, ctx->pinned[s], len, hipMemcpyHostToDevice, stream));
        ZN_HIP_TRY(ctx, hipEventRecord(ctx->pinned_done[s], stream));
    }
    fence.done = true;  // the last DMAs may run on; pinned_done orders the ring's reuse
    return ZN_OK;
}

// Device -> host after the work queued on the stream, then wait.  Large
// copies: the DMA of chunk i + 1 runs while chunk i is copied out of its
// pinned buffer.
int copy_out_and_wait(zn_ctx *ctx, float *dst, const float *src, size_t n) {
    if (ctx->capturing) return ZN_ERR_INVALID_ARG;
    const size_t bytes = n * sizeof(float);
    if (bytes < kStageMin) {
        if (n) ZN_HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
        ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        return ZN_OK;
    }
    int rc = ensure_staging(ctx);
    if (rc) return rc;
    PinnedFence fence{ctx};
    const size_t chunks = (bytes + kStageBytes - 1) / kStageBytes;
    auto issue = [&](size_t i) -> int {
        const size_t off = i * kStageBytes, len = std::min(kStageBytes, bytes - off);
        const int s = (int)(i & 1);
        ZN_HIP_TRY(ctx, hipMemcpyAsync(ctx->pinned[s], (const char *)src + off, len, hipMemcpyDeviceToHost,
                                       ctx->stream));
        ZN_HIP_TRY(ctx, hipEventRecord(ctx->pinned_done[s], ctx->stream));
        return ZN_OK;
    };
    if ((rc = issue(0))) return rc;
    for (size_t i = 0; i < chunks; ++i) {
        // buffer (i + 1) % 2 was drained by this host thread in step i - 1
        if (i + 1 < chunks && (rc = issue(i + 1))) return rc;
        const int s = (int)(i & 1);
        ZN_HIP_TRY(ctx, hipEventSynchronize(ctx->pinned_done[s]));
        const size_t off = i * kStageBytes, len = std::min(kStageBytes, bytes - off);
        ctx->copier->copy((char *)dst + off, ctx->pinned[s], len);
    }
    ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    fence.done = true;
    return ZN_OK;
}

void release_pipeline(zn_ctx *ctx) {
    if (ctx->up) (void)hipStreamSynchronize(ctx->up);
    if (ctx->down) (void)hipStreamSynchronize(ctx->down);
    for (int i = 0; i < 2; ++i) {
        if (ctx->pinned_out_done[i]) (void)hipEventDestroy(ctx->pinned_out_done[i]);
        if (ctx->pinned_out[i]) (void)hipHostFree(ctx->pinned_out[i]);
        if (ctx->chunk_in[i]) (void)hipEventDestroy(ctx->chunk_in[i]);
        if (ctx->chunk_out[i]) (void)hipEventDestroy(ctx->chunk_out[i]);
        ctx->pinned_out_done[i] = ctx->chunk_in[i] = ctx->chunk_out[i] = nullptr;
        ctx->pinned_out[i] = nullptr;
    }
    if (ctx->entry) (void)hipEventDestroy(ctx->entry);
    ctx->entry = nullptr;
    if (ctx->up) (void)hipStreamDestroy(ctx->up);
    if (ctx->down) (void)hipStreamDestroy(ctx->down);
    ctx->up = ctx->down = nullptr;
}

// Ready only when complete (the upload stream is made last); a failed
// set-up releases what it made.
int ensure_pipeline(zn_ctx *ctx) {
    int rc = ensure_staging(ctx);
    if (rc) return rc;
    if (ctx->up) return ZN_OK;
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        const int s0 = 11 + 4 * i;
        e = setup_step(s0, hipHostMalloc((void **)&ctx->pinned_out[i], kStageBytes, hipHostMallocDefault));
        if (e == hipSuccess)
            e = setup_step(s0 + 1, hipEventCreateWithFlags(&ctx->pinned_out_done[i], hipEventDisableTiming));
        if (e == hipSuccess) e = setup_step(s0 + 2, hipEventCreateWithFlags(&ctx->chunk_in[i], hipEventDisableTiming));
        if (e == hipSuccess) e = setup_step(s0 + 3, hipEventCreateWithFlags(&ctx->chunk_out[i], hipEventDisableTiming));
    }
    if (e == hipSuccess) e = setup_step(19, hipEventCreateWithFlags(&ctx->entry, hipEventDisableTiming));
    if (e == hipSuccess) e = setup_step(20, hipStreamCreateWithFlags(&ctx->down, hipStreamNonBlocking));
    hipStream_t up = nullptr;
    if (e == hipSuccess) e = setup_step(21, hipStreamCreateWithFlags(&up, hipStreamNonBlocking));
    if (e != hipSuccess) {
        if (up) (void)hipStreamDestroy(up);
        release_pipeline(ctx);
        return fail_hip(ctx, e, e == hipErrorOutOfMemory ? ZN_ERR_OOM : ZN_ERR_HIP);
    }
    ctx->up = up;
    return ZN_OK;
}

// One step of the chunked host GEMM's transfers: `ups` (host -> device, on
// the upload stream through the staging ring) and `downs` (device -> host,
// on the download stream through the download ring, after the download
// stream's pending waits) are cut into ring-sized pieces and interleaved, so
// both DMA directions run at once while this thread copies host memory in
// and out of the pinned rings.  Returns when every download piece is in host
// memory; uploads are only queued.
struct Span {
    char *dst;
    const char *src;
    size_t bytes;
};

int transfer_step(zn_ctx *ctx, const std::vector<Span> &ups, const std::vector<Span> &downs) {
    struct Piece {
        char *dst;
        const char *src;
        size_t len;
    };
    auto cut = [](const std::vector<Span> &spans) {
        std::vector<Piece> out;
        for (const Span &sp : spans)
            for (size_t off = 0; off < sp.bytes; off += kStageBytes)
                out.push_back({sp.dst + off, sp.src + off, std::min(kStageBytes, sp.bytes - off)});
        return out;
    };
    const std::vector<Piece> up = cut(ups), down = cut(downs);
    auto issue_down = [&](size_t d) -> int {
        const int s = (int)(d & 1);
        ZN_HIP_TRY(ctx, hipMemcpyAsync(ctx->pinned_out[s], down[d].src, down[d].len, hipMemcpyDeviceToHost, ctx->down));
        ZN_HIP_TRY(ctx, hipEventRecord(ctx->pinned_out_done[s], ctx->down));
        return ZN_OK;
    };
    int rc;
    for (size_t d = 0; d < std::min<size_t>(2, down.size()); ++d)
        if ((rc = issue_down(d))) return rc;
    // Whichever side is ready goes next (non-blocking event queries), so a
    // download that waits for its GEMM does not hold up the uploads; when
    // neither is ready, block on the upload buffer (uploads gate the next
    // GEMM) or else on the download.
    auto ready = [&](hipEvent_t e, bool &yes) -> int {
        const hipError_t q = hipEventQuery(e);
        if (q != hipSuccess && q != hipErrorNotReady) return fail_hip(ctx, q);
        yes = q == hipSuccess;
        return ZN_OK;
    };
    for (size_t u = 0, d = 0; u < up.size() || d < down.size();) {
        bool up_ready = false, down_ready = false;
        if (u < up.size() && (rc = ready(ctx->pinned_done[u & 1], up_ready))) return rc;
        if (d < down.size() && (rc = ready(ctx->pinned_out_done[d & 1], down_ready))) return rc;
        if (!up_ready && !down_ready) {
            if (u < up.size()) {
                ZN_HIP_TRY(ctx, hipEventSynchronize(ctx->pinned_done[u & 1]));  // its previous DMA has read it
                up_ready = true;
            } else {
                ZN_HIP_TRY(ctx, hipEventSynchronize(ctx->pinned_out_done[d & 1]));
                down_ready = true;
            }
        }
        if (up_ready) {
            const int s = (int)(u & 1);
            ctx->copier->copy(ctx->pinned[s], up[u].src, up[u].len);
            ZN_HIP_TRY(ctx, hipMemcpyAsync(up[u].dst, ctx->pinned[s], up[u].len, hipMemcpyHostToDevice, ctx->up));
            ZN_HIP_TRY(ctx, hipEventRecord(ctx->pinned_done[s], ctx->up));
            ++u;
        }
        if (down_ready) {
            const int s = (int)(d & 1);
            ctx->copier->copy(down[d].dst, ctx->pinned_out[s], down[d].len);
            if (d + 2 < down.size() && (rc = issue_down(d + 2))) return rc;  // into the buffer just drained
            ++d;
        }
    }
    return ZN_OK;
}

// Host-slice GEMM in row chunks of A and C (NN and NT, whose A chunks are
// contiguous rows), so that PCIe transfers overlap the GEMM: B (and the
// bias) go up first on the upload stream; then A chunk i + 1 (and C chunk
// i + 1 when accumulating) goes up while the context stream multiplies
// chunk i and C chunk i - 1 comes down on the download stream (PCIe is full
// duplex; transfer_step interleaves the two directions).  Each chunk is an
// ordinary GEMM of `rows` rows on the device buffers, so the row results are
// those of the unchunked call whenever both run unsplit (split-K changes only
// the order of K partial sums).
int host_gemm_chunked(zn_ctx *ctx, int layout, const float *a, const float *b, const float *bias, float *c, size_t m,
                      size_t n, size_t k, int accumulate, int act, float *da, float *db, float *dc, float *dbias,
                      size_t rows) {
    int rc = ensure_pipeline(ctx);
    if (rc) return rc;
    // device buffers from the pool may still be read by work queued on the
    // context stream: the side streams start after it
    ZN_HIP_TRY(ctx, hipEventRecord(ctx->entry, ctx->stream));
    ZN_HIP_TRY(ctx, hipStreamWaitEvent(ctx->up, ctx->entry, 0));
    ZN_HIP_TRY(ctx, hipStreamWaitEvent(ctx->down, ctx->entry, 0));
    if ((rc = copy_in(ctx, db, b, k * n, ctx->up))) return rc;
    if (bias && (rc = copy_in(ctx, dbias, bias, n, ctx->up))) return rc;
    const size_t chunks = (m + rows - 1) / rows;
    auto first = [&](size_t i) { return i * rows; };
    auto count = [&](size_t i) { return std::min(rows, m - i * rows); };
    auto ups = [&](size_t i) {
        std::vector<Span> v{{(char *)(da + first(i) * k), (const char *)(a + first(i) * k), count(i) * k * sizeof(float)}};
        if (accumulate)
            v.push_back({(char *)(dc + first(i) * n), (const char *)(c + first(i) * n), count(i) * n * sizeof(float)});
        return v;
    };
    auto downs = [&](size_t i) {
        return std::vector<Span>{
            {(char *)(c + first(i) * n), (const char *)(dc + first(i) * n), count(i) * n * sizeof(float)}};
    };
    const int64_t ldb = layout == ZN_LAYOUT_NT ? (int64_t)k : (int64_t)n;
    if ((rc = transfer_step(ctx, ups(0), {}))) return rc;
    ZN_HIP_TRY(ctx, hipEventRecord(ctx->chunk_in[0], ctx->up));
    for (size_t i = 0; i < chunks; ++i) {
        ZN_HIP_TRY(ctx, hipStreamWaitEvent(ctx->stream, ctx->chunk_in[i & 1], 0));
        rc = gemm_launch(ctx, layout, (int64_t)count(i), (int64_t)n, (int64_t)k, da + first(i) * k, (int64_t)k, 0,
                         db, ldb, 0, dc + first(i) * n, (int64_t)n, 0, 1, accumulate, bias ? dbias : nullptr, act);
        if (rc) return rc;
        ZN_HIP_TRY(ctx, hipEventRecord(ctx->chunk_out[i & 1], ctx->stream));
        if (i >= 1) ZN_HIP_TRY(ctx, hipStreamWaitEvent(ctx->down, ctx->chunk_out[(i - 1) & 1], 0));
        if ((rc = transfer_step(ctx, i + 1 < chunks ? ups(i + 1) : std::vector<Span>{},
                                i >= 1 ? downs(i - 1) : std::vector<Span>{})))
            return rc;
        if (i + 1 < chunks) ZN_HIP_TRY(ctx, hipEventRecord(ctx->chunk_in[(i + 1) & 1], ctx->up));
    }
    ZN_HIP_TRY(ctx, hipStreamWaitEvent(ctx->down, ctx->chunk_out[(chunks - 1) & 1], 0));
    if ((rc = transfer_step(ctx, {}, downs(chunks - 1)))) return rc;
    ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->down));
    ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->up));
    ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return ZN_OK;
}

// Small host-slice calls.  Every synchronous DMA costs ~10 us of latency on
// MI355X whatever its size below ~128 KiB, and a pageable copy more (128 KiB:
// 35 us H2D against 10 us pinned), so small calls stage through the pinned
// buffer: the inputs are copied into it back to back and go up in one DMA,
// and results of at most kZeroCopyBytes are written by the kernel straight
// into the pinned buffer (device-accessible host memory), with no download.
// A 128 KiB elementwise call measured 36.6 us with pageable copies and 20.4 us
// zero-copy.  Host-slice calls are synchronous, so the pinned buffer is free
// on entry.
constexpr size_t kSmallHostBytes = (size_t)4 << 20;  // inputs and outputs of a small call
constexpr size_t kZeroCopyBytes = (size_t)1 << 20;  // GEMM outputs written straight to pinned memory
// Streaming elementwise kernels (every element read and written once, many
// loads in flight) run on the pinned block directly up to this size: 1 MiB
// measured 123 us zero-copy against 136 us with copies.  Kernels whose
// threads walk long dependent chains of loads (the column sums of
// accumulateBias) do not: each host-memory load costs a PCIe round trip.
constexpr size_t kZeroCopyStreamBytes = (size_t)1 << 20;

// 256-byte-aligned regions of the first pinned staging buffer.
struct PinnedBlock {
    float *base;
    size_t used = 0;  // floats
    float *take(size_t n) {
        float *q = base + used;
        used += (n + 63) & ~(size_t)63;
        return q;
    }
};

// Host-slice GEMM: stage A, B (and C when accumulating), run, download C.
// Large NN/NT problems go through host_gemm_chunked, small ones through one
// pinned block.
int host_gemm(zn_ctx *ctx, int layout, const float *a, size_t a_len, const float *b, size_t b_len, const float *bias,
              size_t bias_len, float *c, size_t c_len, size_t m, size_t n, size_t k, int accumulate, int act) {
    if (!ctx) return ZN_ERR_INVALID_ARG;
    size_t mk, kn, mn;
    if (!mul_ok(m, k, &mk) || !mul_ok(k, n, &kn) || !mul_ok(m, n, &mn)) return ZN_ERR_OVERFLOW;
    if (m > INT_MAX || n > INT_MAX || k > INT_MAX) return ZN_ERR_OVERFLOW;
    if (a_len < mk || b_len < kn || c_len < mn) return ZN_ERR_INVALID_ARG;
    if ((mk && !a) || (kn && !b) || (mn && !c)) return ZN_ERR_INVALID_ARG;
    if (bias && bias_len < n) return ZN_ERR_INVALID_ARG;
    if (mn == 0) return ZN_OK;
    if (ctx->capturing) return ZN_ERR_INVALID_ARG;  // host-slice calls read and write host memory synchronously
    int rc = select_device(ctx);
    if (rc) return rc;
    const int64_t lda = layout == ZN_LAYOUT_TN ? (int64_t)m : (int64_t)k;
    const int64_t ldb = layout == ZN_LAYOUT_NT ? (int64_t)k : (int64_t)n;
    if ((mk + kn + (bias ? n : 0) + mn) * sizeof(float) <= kSmallHostBytes) {
        if ((rc = ensure_staging(ctx))) return rc;
        PinnedBlock pb{ctx->pinned[0]};
        float *pa = pb.take(mk), *pbm = pb.take(kn), *pbias = bias ? pb.take(n) : nullptr;
        const size_t in_floats = pb.used;
        float *pc = pb.take(mn);
        std::memcpy(pa, a, mk * sizeof(float));
        std::memcpy(pbm, b, kn * sizeof(float));
        if (bias) std::memcpy(pbias, bias, n * sizeof(float));
        if (accumulate) std::memcpy(pc, c, mn * sizeof(float));
        Lease din(ctx), dc(ctx);
        PinnedFence fence{ctx};
        if ((rc = din.get(in_floats))) return rc;
        ZN_HIP_TRY(ctx, hipMemcpyAsync(din.ptr, pa, in_floats * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
        const bool zero_copy = mn * sizeof(float) <= kZeroCopyBytes;
        float *cdev = pc;  // zero-copy: the kernels read C_old from and write C to the pinned block
        if (!zero_copy) {
            if ((rc = dc.get(mn))) return rc;
            cdev = dc.ptr;
            if (accumulate)
                ZN_HIP_TRY(ctx, hipMemcpyAsync(dc.ptr, pc, mn * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
        }
        rc = gemm_launch(ctx, layout, (int64_t)m, (int64_t)n, (int64_t)k, din.ptr, lda > 0 ? lda : 1, 0,
                         din.ptr + (pbm - pa), ldb > 0 ? ldb : 1, 0, cdev, (int64_t)n, 0, 1, accumulate,
                         bias ? din.ptr + (pbias - pa) : nullptr, act);
        if (rc) return rc;
        if (!zero_copy)
            ZN_HIP_TRY(ctx, hipMemcpyAsync(pc, dc.ptr, mn * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
        ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        fence.done = true;
        std::memcpy(c, pc, mn * sizeof(float));
        return ZN_OK;
    }
    Lease da(ctx), db(ctx), dc(ctx), dbias(ctx);
    if ((rc = da.get(mk)) || (rc = db.get(kn)) || (rc = dc.get(mn))) return rc;
    if (bias && (rc = dbias.get(n))) return rc;
    // Row chunks of about a quarter of A, 8 to 64 MiB, whole multiples of 256 rows, at least two,
    // of nearly equal size
    constexpr size_t kChunkMin = (size_t)8 << 20, kChunkMax = (size_t)64 << 20;
    const size_t a_bytes = mk * sizeof(float);
    if ((layout == ZN_LAYOUT_NN || layout == ZN_LAYOUT_NT) && k > 0 && a_bytes >= 2 * kChunkMin && m >= 512) {
        const size_t target = std::min(kChunkMax, std::max(kChunkMin, a_bytes / 4));
        size_t rows = std::max<size_t>(256, target / (k * sizeof(float)) / 256 * 256);
        const size_t chunks = (m + rows - 1) / rows;
        rows = ((m + chunks - 1) / chunks + 255) / 256 * 256;  // balanced: no small last chunk
        if (rows < m) {
            rc = host_gemm_chunked(ctx, layout, a, b, bias, c, m, n, k, accumulate, act, da.ptr, db.ptr, dc.ptr,
                                   bias ? dbias.ptr : nullptr, rows);
            if (rc && ctx->up) {  // nothing may still use the leased buffers when they go back to the pool
                (void)hipStreamSynchronize(ctx->up);
                (void)hipStreamSynchronize(ctx->down);
                (void)hipStreamSynchronize(ctx->stream);
            }
            return rc;
        }
    }
    if ((rc = copy_in(ctx, da.ptr, a, mk)) || (rc = copy_in(ctx, db.ptr, b, kn))) return rc;
    if (accumulate && (rc = copy_in(ctx, dc.ptr, c, mn))) return rc;
    if (bias && (rc = copy_in(ctx, dbias.ptr, bias, n))) return rc;
    rc = gemm_launch(ctx, layout, (int64_t)m, (int64_t)n, (int64_t)k, da.ptr, lda > 0 ? lda : 1, 0, db.ptr,
                     ldb > 0 ? ldb : 1, 0, dc.ptr, (int64_t)n, 0, 1, accumulate, bias ? dbias.ptr : nullptr, act);
    if (rc) return rc;
    return copy_out_and_wait(ctx, c, dc.ptr, mn);
}

}  // namespace

// =================================================================== C ABI
extern "C" {

int zn_hip_abi_version(void) { return ZN_HIP_ABI_VERSION; }

int zn_hip_available(void) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return count > 0 ? 1 : 0;
}

const char *zn_hip_status_string(int status) {
    switch (status) {
    case ZN_OK: return "ZN_OK";
    case ZN_ERR_NO_DEVICE: return "ZN_ERR_NO_DEVICE: no usable gfx950 HIP device";
    case ZN_ERR_CODE_OBJECT: return "ZN_ERR_CODE_OBJECT: gfx950 code object missing or not loadable";
    case ZN_ERR_SYMBOL: return "ZN_ERR_SYMBOL: kernel symbol missing from the code object";
    case ZN_ERR_INVALID_ARG: return "ZN_ERR_INVALID_ARG: invalid argument";
    case ZN_ERR_OOM: return "ZN_ERR_OOM: device allocation failed";
    case ZN_ERR_LAUNCH: return "ZN_ERR_LAUNCH: kernel launch failed";
    case ZN_ERR_HIP: return "ZN_ERR_HIP: HIP runtime error";
    case ZN_ERR_OVERFLOW: return "ZN_ERR_OVERFLOW: size overflow or beyond 32-bit index range";
    default: return "ZN_ERR_UNKNOWN";
    }
}

int zn_hip_create(int device, const char *code_object_dir, zn_ctx **out) {
    if (!out) return ZN_ERR_INVALID_ARG;
    *out = nullptr;
    std::string dir;
    if (code_object_dir && *code_object_dir)
        dir = code_object_dir;
    else if (const char *env = std::getenv("ZN_HIP_CODE_OBJECT_DIR"))
        dir = env;
    else
        dir = library_dir();
    const std::string gemm_path = dir + "/" + kGemmObject;
    const std::string conv_path = dir + "/" + kConvObject;
    const std::string elt_path = dir + "/" + kEltObject;
    const std::string attn_path = dir + "/" + kAttnObject;
    const std::string mlp_path = dir + "/" + kMlpObject;
    // The code objects are checked on the host first, so a bad directory is
    // reported the same way with or without a device.
    for (const std::string *path : {&gemm_path, &conv_path, &elt_path, &attn_path, &mlp_path})
        if (!code_object_ok(*path)) return ZN_ERR_CODE_OBJECT;

    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        return ZN_ERR_NO_DEVICE;
    }
    if (device < 0 || device >= count) return ZN_ERR_INVALID_ARG;

    zn_ctx *ctx = new (std::nothrow) zn_ctx();
    if (!ctx) return ZN_ERR_OOM;
    ctx->device = device;
    auto bail = [&](int rc) {
        zn_hip_destroy(ctx);
        return rc;
    };

    if (hipSetDevice(device) != hipSuccess) return bail(ZN_ERR_NO_DEVICE);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return bail(ZN_ERR_NO_DEVICE);
    std::snprintf(ctx->info.name, sizeof(ctx->info.name), "%s", prop.gcnArchName);
    ctx->info.compute_units = prop.multiProcessorCount;
    ctx->info.clock_khz = prop.clockRate;
    ctx->info.total_mem = (int64_t)prop.totalGlobalMem;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return bail(ZN_ERR_NO_DEVICE);
    // The no-allocation GEMM's scratch: a failure here is kept and reported
    // by zn_hip_sgemm_noalloc; every other entry point works without it.
    (void)resolve_scratch(ctx);

    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) return bail(fail_hip(ctx, e));
    if (hipModuleLoad(&ctx->gemm_module, gemm_path.c_str()) != hipSuccess) {
        ctx->gemm_module = nullptr;
        return bail(ZN_ERR_CODE_OBJECT);
    }
    if (hipModuleLoad(&ctx->conv_module, conv_path.c_str()) != hipSuccess) {
        ctx->conv_module = nullptr;
        return bail(ZN_ERR_CODE_OBJECT);
    }
    if (hipModuleLoad(&ctx->elt_module, elt_path.c_str()) != hipSuccess) {
        ctx->elt_module = nullptr;
        return bail(ZN_ERR_CODE_OBJECT);
    }
    if (hipModuleLoad(&ctx->attn_module, attn_path.c_str()) != hipSuccess) {
        ctx->attn_module = nullptr;
        return bail(ZN_ERR_CODE_OBJECT);
    }
    if (hipModuleLoad(&ctx->mlp_module, mlp_path.c_str()) != hipSuccess) {
        ctx->mlp_module = nullptr;
        return bail(ZN_ERR_CODE_OBJECT);
    }
    for (int l = 0; l < 3; ++l)
        for (int t = 0; t < kNumTiles; ++t)
            for (int v = kTiles[t].plain ? 0 : 1; v < (t == kTileR ? 3 : 2); ++v) {
                char name[64];
                std::snprintf(name, sizeof(name), "zn_sgemm_%s_%s%s", kLayoutName[l], kTiles[t].suffix,
                              v == 2 ? "_u" : v ? "_v" : "");
                if (hipModuleGetFunction(&ctx->gemm[l][t][v], ctx->gemm_module, name) != hipSuccess)
                    return bail(ZN_ERR_SYMBOL);
                int threads = 0;
                if (hipFuncGetAttribute(&threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, ctx->gemm[l][t][v]) !=
                        hipSuccess ||
                    threads < 64 || threads > 1024)
                    return bail(ZN_ERR_SYMBOL);
                ctx->gemm_threads[l][t][v] = threads;
            }
    for (int t = 0; t < kNumTiles; ++t)
        for (int v = 0; v < 2 && kTiles[t].conv; ++v)
            for (int g = 0; g < 2; ++g) {
                char name[64];
                std::snprintf(name, sizeof(name), "zn_conv_nn_%s%s%s", kTiles[t].suffix, v ? "_v" : "", g ? "_g" : "");
                if (hipModuleGetFunction(&ctx->conv[t][v][g], ctx->conv_module, name) != hipSuccess)
                    return bail(ZN_ERR_SYMBOL);
            }
    for (int t = 0; t < kNumTiles; ++t)
        for (int v = 0; v < 2 && kTiles[t].conv; ++v) {
            char name[64];
            std::snprintf(name, sizeof(name), "zn_convt_nt_%s%s", kTiles[t].suffix, v ? "_v" : "");
            if (hipModuleGetFunction(&ctx->convt[t][v], ctx->conv_module, name) != hipSuccess)
                return bail(ZN_ERR_SYMBOL);
            int occ = 0;
            if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&occ, ctx->convt[t][v], kTiles[t].threads, 0) !=
                    hipSuccess ||
                occ < 1)
                occ = 1;
            ctx->convt_occ[t][v] = occ;
            std::snprintf(name, sizeof(name), "zn_convw_tn_%s%s", kTiles[t].suffix, v ? "_v" : "");
            if (hipModuleGetFunction(&ctx->convw[t][v], ctx->conv_module, name) != hipSuccess)
                return bail(ZN_ERR_SYMBOL);
            std::snprintf(name, sizeof(name), "zn_convf_nt_%s%s", kTiles[t].suffix, v ? "_v" : "");
            if (hipModuleGetFunction(&ctx->convf[t][v], ctx->conv_module, name) != hipSuccess)
                return bail(ZN_ERR_SYMBOL);
            std::snprintf(name, sizeof(name), "zn_convwn_tn_%s%s", kTiles[t].suffix, v ? "_v" : "");
            if (hipModuleGetFunction(&ctx->convwn[t][v], ctx->conv_module, name) != hipSuccess)
                return bail(ZN_ERR_SYMBOL);
        }
    // the 128x128 tile's only convolution kernel: the NHWC weight gradient, 16-byte rows
    if (hipModuleGetFunction(&ctx->convwn[kTileR][1], ctx->conv_module, "zn_convwn_tn_r_v") != hipSuccess)
        return bail(ZN_ERR_SYMBOL);
    for (int l = 0; l < 3; ++l)
        for (int w = 0; w < 2; ++w)
            for (int v = 0; v < 2; ++v) {
                char name[64];
                std::snprintf(name, sizeof(name), "zn_sgemmk%d_%s%s", w ? 8 : 4, kLayoutName[l], v ? "_v" : "");
                if (hipModuleGetFunction(&ctx->gemmk[l][w][v], ctx->gemm_module, name) != hipSuccess)
                    return bail(ZN_ERR_SYMBOL);
            }
    for (int l = 0; l < 3; ++l)
        for (int v = 0; v < 2; ++v) {
            char name[64];
            std::snprintf(name, sizeof(name), "zn_sgemmk4s_%s%s", kLayoutName[l], v ? "_v" : "");
            if (hipModuleGetFunction(&ctx->gemmks[l][v], ctx->gemm_module, name) != hipSuccess)
                return bail(ZN_ERR_SYMBOL);
            for (int r = 0; r < 3; ++r) {
                std::snprintf(name, sizeof(name), "zn_sgemmq%s_%s%s", r == 2 ? "8" : r ? "4m" : "4", kLayoutName[l],
                              v ? "_v" : "");
                if (hipModuleGetFunction(&ctx->gemmq[l][r][v], ctx->gemm_module, name) != hipSuccess)
                    return bail(ZN_ERR_SYMBOL);
                int threads = 0;
                if (hipFuncGetAttribute(&threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, ctx->gemmq[l][r][v]) !=
                        hipSuccess ||
                    (threads != 256 && threads != 512))
                    return bail(ZN_ERR_SYMBOL);
                ctx->gemmq_threads[l][r][v] = threads;
            }
        }
    for (int l = 0; l < 3; ++l)
        for (int t = 0; t < kNumTiles; ++t) {
            if (!kTiles[t].persistent) continue;
            char name[64];
            std::snprintf(name, sizeof(name), "zn_sgemmp_%s_%s_v", kLayoutName[l], kTiles[t].suffix);
            if (hipModuleGetFunction(&ctx->gemmp[l][t], ctx->gemm_module, name) != hipSuccess)
                return bail(ZN_ERR_SYMBOL);
            int occ = 0;
            if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&occ, ctx->gemmp[l][t], kTiles[t].threads, 0) !=
                    hipSuccess ||
                occ < 1)
                occ = 1;
            ctx->gemmp_occ[l][t] = occ;
        }
    for (int l = 0; l < 3; ++l) {
        char name[64];
        std::snprintf(name, sizeof(name), "zn_sgemmpd_%s_l_v", kLayoutName[l]);
        if (hipModuleGetFunction(&ctx->gemmpd[l], ctx->gemm_module, name) != hipSuccess) return bail(ZN_ERR_SYMBOL);
        std::snprintf(name, sizeof(name), "zn_sgemmpd4_%s_l_v", kLayoutName[l]);
        if (hipModuleGetFunction(&ctx->gemmpd4[l], ctx->gemm_module, name) != hipSuccess) return bail(ZN_ERR_SYMBOL);
        int threads = 0, occ = 0;
        if (hipFuncGetAttribute(&threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, ctx->gemmpd[l]) != hipSuccess ||
            threads < 64)
            return bail(ZN_ERR_SYMBOL);
        if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&occ, ctx->gemmpd[l], threads, 0) != hipSuccess ||
            occ < 1)
            occ = 1;
        ctx->gemmpd_threads[l] = threads;
        ctx->gemmpd_occ[l] = occ;
    }
    if (hipModuleGetFunction(&ctx->splitk_reduce, ctx->gemm_module, "zn_splitk_reduce") != hipSuccess ||
        hipModuleGetFunction(&ctx->dense_bwd[0], ctx->gemm_module, "zn_dense_bwd_m") != hipSuccess ||
        hipModuleGetFunction(&ctx->dense_bwd[1], ctx->gemm_module, "zn_dense_bwd_m_v") != hipSuccess ||
        hipModuleGetFunction(&ctx->dense_bwd_k[0], ctx->gemm_module, "zn_dense_bwd_k") != hipSuccess ||
        hipModuleGetFunction(&ctx->dense_bwd_k[1], ctx->gemm_module, "zn_dense_bwd_k_v") != hipSuccess)
        return bail(ZN_ERR_SYMBOL);
    for (int i = 0; i < kNumElt; ++i)
        if (hipModuleGetFunction(&ctx->elt[i], ctx->elt_module, kEltName[i]) != hipSuccess) return bail(ZN_ERR_SYMBOL);
    if (hipModuleGetFunction(&ctx->pair_fwd[0], ctx->mlp_module, "zn_dense_pair_fwd") != hipSuccess ||
        hipModuleGetFunction(&ctx->pair_fwd[1], ctx->mlp_module, "zn_dense_pair_fwd_v") != hipSuccess)
        return bail(ZN_ERR_SYMBOL);
    for (int v = 0; v < 2; ++v) {
        int threads = 0;
        if (hipFuncGetAttribute(&threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, ctx->pair_fwd[v]) != hipSuccess ||
            (threads != 256 && threads != 512 && threads != 1024))
            return bail(ZN_ERR_SYMBOL);
        ctx->pair_fwd_threads[v] = threads;
    }
    for (int a1 = 0; a1 < 4; ++a1)
        for (int a2 = 0; a2 < 2; ++a2)
            for (int v = 0; v < 2; ++v) {
                char name[64];
                std::snprintf(name, sizeof(name), "zn_dense_pair_bwd_%d%d%s", a1, a2, v ? "_v" : "");
                if (hipModuleGetFunction(&ctx->pair_bwd[a1][a2][v], ctx->mlp_module, name) != hipSuccess)
                    return bail(ZN_ERR_SYMBOL);
            }
    for (int d = 0; d < 3; ++d)
        for (int v = 0; v < 2; ++v) {
            char name[64];
            std::snprintf(name, sizeof(name), "zn_attention_d%d%s", kAttnDims[d], v ? "_v" : "");
            if (hipModuleGetFunction(&ctx->attn[d][v], ctx->attn_module, name) != hipSuccess) return bail(ZN_ERR_SYMBOL);
        }
    void *counters = nullptr;
    if ((e = hipMalloc(&counters, kCounterSlots * kCounterStride * sizeof(int32_t))) != hipSuccess) {
        (void)hipGetLastError();
        return bail(fail_hip(ctx, e, ZN_ERR_OOM));
    }
    ctx->counters = static_cast<int32_t *>(counters);
    if ((e = hipMemset(counters, 0, kCounterSlots * kCounterStride * sizeof(int32_t))) != hipSuccess)
        return bail(fail_hip(ctx, e));
    *out = ctx;
    return ZN_OK;
}

int zn_hip_destroy(zn_ctx *ctx) {
    if (!ctx) return ZN_OK;
    if (ctx->device >= 0) (void)hipSetDevice(ctx->device);
    if (ctx->capturing) {  // abandon an open capture
        hipGraph_t g = nullptr;
        if (hipStreamEndCapture(ctx->stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
        (void)hipGetLastError();
        ctx->capturing = false;
        for (auto &b : ctx->captured) ctx->pool[b.second].push_back(b.first);
        ctx->captured.clear();
    }
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    forget_scratch_owner(ctx);
    release_pipeline(ctx);
    release_staging(ctx);
    while (!ctx->graphs.empty()) (void)zn_hip_graph_destroy(ctx->graphs.back());
    for (void *w : ctx->retired_ws) (void)hipFree(w);
    ctx->retired_ws.clear();
    for (auto &kv : ctx->pool)
        for (void *p : kv.second) (void)hipFree(p);
    ctx->pool.clear();
    if (ctx->ws) (void)hipFree(ctx->ws);
    ctx->ws = nullptr;
    if (ctx->counters) (void)hipFree(ctx->counters);
    ctx->counters = nullptr;
    if (ctx->gemm_module) (void)hipModuleUnload(ctx->gemm_module);
    if (ctx->conv_module) (void)hipModuleUnload(ctx->conv_module);
    if (ctx->elt_module) (void)hipModuleUnload(ctx->elt_module);
    if (ctx->attn_module) (void)hipModuleUnload(ctx->attn_module);
    if (ctx->mlp_module) (void)hipModuleUnload(ctx->mlp_module);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    (void)hipGetLastError();
    delete ctx;
    return ZN_OK;
}

int zn_hip_last_hip_error(const zn_ctx *ctx) { return ctx ? ctx->last_hip_error : 0; }

int zn_hip_device_info(const zn_ctx *ctx, zn_device_info *out) {
    if (!ctx || !out) return ZN_ERR_INVALID_ARG;
    *out = ctx->info;
    return ZN_OK;
}

void *zn_hip_stream(const zn_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

// ----------------------------------------------------------------- memory
int zn_hip_alloc(zn_ctx *ctx, size_t bytes, void **out) {
    if (!ctx || !out) return ZN_ERR_INVALID_ARG;
    *out = nullptr;
    int rc = select_device(ctx);
    if (rc) return rc;
    hipError_t e = hipMalloc(out, bytes ? bytes : 4);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *out = nullptr;
        return fail_hip(ctx, e, ZN_ERR_OOM);
    }
    return ZN_OK;
}

int zn_hip_free(zn_ctx *ctx, void *ptr) {
    if (!ctx) return ZN_ERR_INVALID_ARG;
    if (!ptr) return ZN_OK;
    if (ctx->capturing) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    ZN_HIP_TRY(ctx, hipFree(ptr));
    return ZN_OK;
}

static int zn_copy(zn_ctx *ctx, void *dst, const void *src, size_t bytes, hipMemcpyKind kind, bool wait) {
    if (!ctx) return ZN_ERR_INVALID_ARG;
    if (bytes == 0) return ZN_OK;
    if (!dst || !src || (wait && ctx->capturing)) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    ZN_HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, kind, ctx->stream));
    if (wait) ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return ZN_OK;
}

int zn_hip_h2d(zn_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return zn_copy(ctx, dst, src, bytes, hipMemcpyHostToDevice, true);
}
int zn_hip_d2h(zn_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return zn_copy(ctx, dst, src, bytes, hipMemcpyDeviceToHost, true);
}
int zn_hip_h2d_async(zn_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return zn_copy(ctx, dst, src, bytes, hipMemcpyHostToDevice, false);
}
int zn_hip_d2h_async(zn_ctx *ctx, void *dst, const void *src, size_t bytes) {
    return zn_copy(ctx, dst, src, bytes, hipMemcpyDeviceToHost, false);
}

int zn_hip_fill_f32(zn_ctx *ctx, float *dst, float value, int64_t count) {
    if (!ctx || count < 0) return ZN_ERR_INVALID_ARG;
    if (count == 0) return ZN_OK;
    if (!dst) return ZN_ERR_INVALID_ARG;
    ZnEltArgs a = {};
    a.out = dst;
    a.rows = 1;
    a.n = count;
    a.value = value;
    return elt_launch(ctx, kFill, count, a);
}

int zn_hip_copy_f32(zn_ctx *ctx, float *dst, const float *src, int64_t count) {
    if (!ctx || count < 0) return ZN_ERR_INVALID_ARG;
    if (count == 0) return ZN_OK;
    if (!dst || !src) return ZN_ERR_INVALID_ARG;
    ZnEltArgs a = {};
    a.out = dst;
    a.in0 = src;
    a.rows = 1;
    a.n = count;
    return elt_launch(ctx, kCopy, (count + 3) / 4, a);
}

int zn_hip_hold_stream(zn_ctx *ctx, float microseconds) {
    if (!ctx || !(microseconds >= 0.0f) || microseconds > 100000.0f) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    ZnEltArgs a = {};
    a.value = microseconds;
    // one sleep of 8 x 64 clocks is at least 0.2 us below 2.6 GHz: the cap
    // is several times the requested wait
    a.n = (int64_t)(microseconds * 20.0f) + 64;
    return launch(ctx, ctx->elt[kHold], 1, 1, 64, &a);
}

int zn_hip_sync(zn_ctx *ctx) {
    if (!ctx || ctx->capturing) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return ZN_OK;
}

// ----------------------------------------------------------------- graphs
int zn_hip_graph_begin(zn_ctx *ctx) {
    if (!ctx || ctx->capturing) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    ZN_HIP_TRY(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed));
    ctx->capturing = true;
    ctx->captured.clear();
    return ZN_OK;
}

int zn_hip_graph_end(zn_ctx *ctx, zn_graph **out) {
    if (!ctx || !out || !ctx->capturing) return ZN_ERR_INVALID_ARG;
    *out = nullptr;
    int rc = select_device(ctx);
    if (rc) return rc;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    ctx->capturing = false;
    std::vector<std::pair<void *, size_t>> bufs;
    bufs.swap(ctx->captured);
    auto give_back = [&]() {
        for (auto &b : bufs) ctx->pool[b.second].push_back(b.first);
    };
    if (e != hipSuccess || !g) {
        give_back();
        return fail_hip(ctx, e != hipSuccess ? e : hipErrorUnknown);
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        give_back();
        return fail_hip(ctx, e);
    }
    zn_graph *graph = new (std::nothrow) zn_graph();
    if (!graph) {
        (void)hipGraphExecDestroy(exec);
        give_back();
        return ZN_ERR_OOM;
    }
    graph->ctx = ctx;
    graph->exec = exec;
    graph->buffers.swap(bufs);
    ctx->graphs.push_back(graph);
    *out = graph;
    return ZN_OK;
}

int zn_hip_graph_launch(zn_ctx *ctx, zn_graph *graph) {
    if (!ctx || !graph || graph->ctx != ctx || ctx->capturing) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    ZN_HIP_TRY(ctx, hipGraphLaunch(graph->exec, ctx->stream));
    return ZN_OK;
}

int zn_hip_graph_destroy(zn_graph *graph) {
    if (!graph) return ZN_OK;
    zn_ctx *ctx = graph->ctx;
    if (ctx->device >= 0) (void)hipSetDevice(ctx->device);
    if (!ctx->capturing) (void)hipStreamSynchronize(ctx->stream);  // replays may still run
    (void)hipGraphExecDestroy(graph->exec);
    for (auto &b : graph->buffers) ctx->pool[b.second].push_back(b.first);
    auto &gs = ctx->graphs;
    gs.erase(std::remove(gs.begin(), gs.end(), graph), gs.end());
    if (gs.empty()) {
        for (void *w : ctx->retired_ws) (void)hipFree(w);
        ctx->retired_ws.clear();
    }
    delete graph;
    return ZN_OK;
}

// ----------------------------------------------------------------- events
int zn_hip_event_create(zn_ctx *ctx, zn_event **out) {
    if (!ctx || !out) return ZN_ERR_INVALID_ARG;
    *out = nullptr;
    int rc = select_device(ctx);
    if (rc) return rc;
    zn_event *ev = new (std::nothrow) zn_event();
    if (!ev) return ZN_ERR_OOM;
    hipError_t e = hipEventCreate(&ev->ev);
    if (e != hipSuccess) {
        delete ev;
        return fail_hip(ctx, e);
    }
    *out = ev;
    return ZN_OK;
}

int zn_hip_event_record(zn_ctx *ctx, zn_event *ev) {
    if (!ctx || !ev) return ZN_ERR_INVALID_ARG;
    ZN_HIP_TRY(ctx, hipEventRecord(ev->ev, ctx->stream));
    return ZN_OK;
}

int zn_hip_event_elapsed_ms(zn_event *start, zn_event *end, float *ms) {
    if (!start || !end || !ms) return ZN_ERR_INVALID_ARG;
    if (hipEventSynchronize(end->ev) != hipSuccess) return ZN_ERR_HIP;
    if (hipEventElapsedTime(ms, start->ev, end->ev) != hipSuccess) return ZN_ERR_HIP;
    return ZN_OK;
}

int zn_hip_event_destroy(zn_event *ev) {
    if (!ev) return ZN_OK;
    (void)hipEventDestroy(ev->ev);
    delete ev;
    return ZN_OK;
}

// ------------------------------------------------------------------ GEMM
int zn_hip_set_gemm_tile(zn_ctx *ctx, int tile) {
    if (!ctx || tile < ZN_TILE_AUTO || tile >= kNumTiles) return ZN_ERR_INVALID_ARG;
    ctx->forced_tile = tile;
    return ZN_OK;
}

int zn_hip_set_gemm_splits(zn_ctx *ctx, int splits) {
    if (!ctx || splits < 0 || splits > 256) return ZN_ERR_INVALID_ARG;
    ctx->forced_splits = splits;
    return ZN_OK;
}

int zn_hip_set_gemm_wave_split(zn_ctx *ctx, int waves) {
    if (!ctx || (waves != -1 && waves != 0 && waves != 4 && waves != 8 && waves != 16)) return ZN_ERR_INVALID_ARG;
    ctx->forced_wave_split = waves;
    return ZN_OK;
}

int zn_hip_set_gemm_persistent(zn_ctx *ctx, int mode) {
    if (!ctx || mode < -1 || mode > 2) return ZN_ERR_INVALID_ARG;
    ctx->forced_persistent = mode;
    return ZN_OK;
}

int zn_hip_sgemm(zn_ctx *ctx, int layout, int64_t m, int64_t n, int64_t k, const float *a, int64_t lda,
                 const float *b, int64_t ldb, float *c, int64_t ldc, int accumulate, const float *bias, int act) {
    return gemm_launch(ctx, layout, m, n, k, a, lda, 0, b, ldb, 0, c, ldc, 0, 1, accumulate, bias, act);
}

int zn_hip_sgemm_noalloc(zn_ctx *ctx, int layout, int64_t m, int64_t n, int64_t k, const float *a, int64_t lda,
                         const float *b, int64_t ldb, float *c, int64_t ldc, int accumulate, const float *bias,
                         int act) {
    if (!ctx) return ZN_ERR_INVALID_ARG;
    if (!ctx->scratch || !ctx->scratch_dev) return ctx->scratch_status != ZN_OK ? ctx->scratch_status : ZN_ERR_HIP;
    ScratchDevice &s = *ctx->scratch_dev;
    std::lock_guard<std::mutex> lock(s.use);
    // Under stream capture the call becomes graph nodes and is not ordered
    // here: whoever replays the graph keeps it apart from other users.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    ZN_HIP_TRY(ctx, hipStreamIsCapturing(ctx->stream, &cap));
    const bool ordered = cap == hipStreamCaptureStatusNone;
    if (ordered && s.recorded && s.owner != ctx) ZN_HIP_TRY(ctx, hipStreamWaitEvent(ctx->stream, s.done, 0));
    int rc;
    {
        NoAllocScope scope(ctx);
        rc = gemm_launch(ctx, layout, m, n, k, a, lda, 0, b, ldb, 0, c, ldc, 0, 1, accumulate, bias, act);
    }
    if (ordered) {
        const hipError_t e = hipEventRecord(s.done, ctx->stream);
        if (e != hipSuccess) {
            // the next user can no longer wait for this call: drain it
            (void)hipGetLastError();
            (void)hipStreamSynchronize(ctx->stream);
            s.recorded = false;
            s.owner = nullptr;
            return rc == ZN_OK ? fail_hip(ctx, e) : rc;
        }
        s.recorded = true;
        s.owner = ctx;
    }
    return rc;
}

int zn_hip_sgemm_strided_batched(zn_ctx *ctx, int layout, int64_t m, int64_t n, int64_t k, const float *a,
                                 int64_t lda, int64_t stride_a, const float *b, int64_t ldb, int64_t stride_b,
                                 float *c, int64_t ldc, int64_t stride_c, int64_t batch, int accumulate,
                                 const float *bias, int act) {
    return gemm_launch(ctx, layout, m, n, k, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c, batch, accumulate,
                       bias, act);
}

// ---------------------------------------------------------- Dense helpers
int zn_hip_add_bias(zn_ctx *ctx, float *out, const float *bias, int64_t rows, int64_t n) {
    if (!ctx || rows < 0 || n < 0) return ZN_ERR_INVALID_ARG;
    if (rows == 0 || n == 0) return ZN_OK;
    if (!out || !bias) return ZN_ERR_INVALID_ARG;
    ZnEltArgs a = {};
    a.out = out;
    a.in0 = bias;
    a.rows = rows;
    a.n = n;
    return elt_launch(ctx, kAddBias, rows * n, a);
}

int zn_hip_activation_forward(zn_ctx *ctx, int act, const float *in, float *out, int64_t len) {
    if (!ctx || len < 0 || act < ZN_ACT_LINEAR || act > ZN_ACT_TANH) return ZN_ERR_INVALID_ARG;
    if (len == 0) return ZN_OK;
    if (!in || !out) return ZN_ERR_INVALID_ARG;
    ZnEltArgs a = {};
    a.out = out;
    a.in0 = in;
    a.rows = 1;
    a.n = len;
    a.act = act;
    return elt_launch(ctx, kActFwd, len, a);
}

int zn_hip_activation_backward(zn_ctx *ctx, int act, const float *y, const float *grad_out, float *grad_in,
                               int64_t len) {
    if (!ctx || len < 0 || act < ZN_ACT_LINEAR || act > ZN_ACT_TANH) return ZN_ERR_INVALID_ARG;
    if (len == 0) return ZN_OK;
    if (!y || !grad_out || !grad_in) return ZN_ERR_INVALID_ARG;
    ZnEltArgs a = {};
    a.out = grad_in;
    a.in0 = y;
    a.in1 = grad_out;
    a.rows = 1;
    a.n = len;
    a.act = act;
    return elt_launch(ctx, kActBwd, len, a);
}

int zn_hip_accumulate_bias(zn_ctx *ctx, float *grad_bias, const float *gaa, int64_t rows, int64_t n) {
    if (!ctx || rows < 0 || n < 0) return ZN_ERR_INVALID_ARG;
    if (rows == 0 || n == 0) return ZN_OK;
    if (!grad_bias || !gaa) return ZN_ERR_INVALID_ARG;
    ZnEltArgs a = {};
    a.out = grad_bias;
    a.in0 = gaa;
    a.rows = rows;
    a.n = n;
    return elt_launch(ctx, kAccBias, n, a);
}

// ------------------------------------------------- conv and attention
static bool conv_dims_ok(int64_t batch, int64_t c, int64_t oc, int64_t kh, int64_t kw, int64_t h, int64_t w,
                         int64_t oh, int64_t ow, int64_t sh, int64_t sw, int64_t ph, int64_t pw) {
    if (batch < 0 || c < 1 || oc < 1 || kh < 1 || kw < 1 || h < 1 || w < 1 || oh < 0 || ow < 0 || sh < 1 ||
        sw < 1 || ph < 0 || pw < 0)
        return false;
    const int64_t lim = INT_MAX;
    return batch <= lim && c * kh * kw <= lim && h * w <= lim && oh * ow <= lim && oc <= lim;
}

static ZnIm2colArgs col_args(float *image, float *col, int64_t batch, int64_t c, int64_t kh, int64_t kw, int64_t h,
                             int64_t w, int64_t oh, int64_t ow, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                             int k_order) {
    ZnIm2colArgs a;
    a.image = image;
    a.col = col;
    a.batch = (int32_t)batch;
    a.channels = (int32_t)c;
    a.in_h = (int32_t)h;
    a.in_w = (int32_t)w;
    a.k_h = (int32_t)kh;
    a.k_w = (int32_t)kw;
    a.out_h = (int32_t)oh;
    a.out_w = (int32_t)ow;
    a.stride_h = (int32_t)sh;
    a.stride_w = (int32_t)sw;
    a.pad_h = (int32_t)ph;
    a.pad_w = (int32_t)pw;
    a.k_order = k_order;
    return a;
}

// zn_im2col: one workgroup per tile of 64 col rows x 64 taps; zn_col2im: one
// per 64 pixels of an input row (grid-stride loops cover the rest).
static int im2col_launch(zn_ctx *ctx, const ZnIm2colArgs &a) {
    const int rc = select_device(ctx);
    if (rc) return rc;
    const int64_t cap = cus_now(ctx) * 32;
    const int64_t units = cdiv((int64_t)a.batch * a.out_h * a.out_w, 64) * cdiv((int64_t)a.k_h * a.k_w * a.channels, 64);
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(units, cap));
    ZnIm2colArgs c = a;
    return launch(ctx, ctx->elt[kIm2col], (unsigned)blocks, 1, 256, &c);
}
static int col2im_launch(zn_ctx *ctx, const ZnIm2colArgs &a) {
    const int rc = select_device(ctx);
    if (rc) return rc;
    const int64_t cap = cus_now(ctx) * 32;
    const int64_t units = (int64_t)a.batch * a.in_h * cdiv(a.in_w, 64);
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(units, cap));
    ZnIm2colArgs c = a;
    return launch(ctx, ctx->elt[kCol2im], (unsigned)blocks, 1, 256, &c);
}

int zn_hip_im2col(zn_ctx *ctx, const float *input, float *col, int64_t batch, int64_t channels, int64_t in_h,
                  int64_t in_w, int64_t k_h, int64_t k_w, int64_t out_h, int64_t out_w, int64_t stride_h,
                  int64_t stride_w, int64_t pad_h, int64_t pad_w) {
    if (!ctx || !conv_dims_ok(batch, channels, 1, k_h, k_w, in_h, in_w, out_h, out_w, stride_h, stride_w, pad_h,
                              pad_w))
        return ZN_ERR_INVALID_ARG;
    const int64_t total = batch * out_h * out_w * k_h * k_w * channels;
    if (total == 0) return ZN_OK;
    if (!input || !col) return ZN_ERR_INVALID_ARG;
    ZnIm2colArgs a = col_args(const_cast<float *>(input), col, batch, channels, k_h, k_w, in_h, in_w, out_h, out_w,
                              stride_h, stride_w, pad_h, pad_w, 0);  // input is only read by zn_im2col
    return im2col_launch(ctx, a);
}

// Implicit-GEMM convolution: per image one NN GEMM
// out_b[OC][OH*OW] = W[OC][K] . im2col(input_b)^T + bias[oc], the im2col
// operand gathered on the fly (no col buffer).  k_order 0 reads W in the
// im2col K order (kh, kw, ic) like cpuConv2dForwardIm2col; 1 reads W as
// [OC][C][kH][kW] like the direct branch of cpuConv2dForward.
static int conv2d_device(zn_ctx *ctx, const float *input, const float *weights, const float *bias, float *output,
                         int64_t batch, int64_t c, int64_t oc, int64_t kh, int64_t kw, int64_t h, int64_t w,
                         int64_t oh, int64_t ow, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int k_order) {
    if (!ctx || !conv_dims_ok(batch, c, oc, kh, kw, h, w, oh, ow, sh, sw, ph, pw)) return ZN_ERR_INVALID_ARG;
    const int64_t hw = oh * ow, kdim = c * kh * kw;
    if (batch == 0 || hw == 0) return ZN_OK;
    if (!input || !weights || !bias || !output) return ZN_ERR_INVALID_ARG;
    if (h * w > INT_MAX || c * h * w > INT_MAX / 4) return ZN_ERR_OVERFLOW;
    ZnConvGeom g = {};
    g.channels = (int32_t)c;
    g.in_h = (int32_t)h;
    g.in_w = (int32_t)w;
    g.k_h = (int32_t)kh;
    g.k_w = (int32_t)kw;
    g.out_w = (int32_t)ow;
    g.stride_h = (int32_t)sh;
    g.stride_w = (int32_t)sw;
    g.pad_h = (int32_t)ph;
    g.pad_w = (int32_t)pw;
    g.k_order = k_order;
    g.div1 = k_order == 0 ? g.channels : g.k_h * g.k_w;
    udiv_magic((uint32_t)g.div1, g.div1_mul, g.div1_shift);
    udiv_magic((uint32_t)g.k_w, g.kw_mul, g.kw_shift);
    udiv_magic((uint32_t)g.out_w, g.ow_mul, g.ow_shift);
    const int64_t plane = c * h * w;
    if (k_order == 0 && c % 4 == 0 && kdim % 4 == 0) {
        // NHWC copy of the images (in chunks of at most 2^28 floats), then an
        // NT GEMM gathering 4 channels per 16-byte load: no partial chunks
        // at the padding, at any stride.
        const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(batch, ((int64_t)1 << 28) / plane));
        Lease nhwc(ctx);
        int rc = nhwc.get((size_t)(chunk * plane));
        if (rc) return rc;
        for (int64_t b0 = 0; b0 < batch; b0 += chunk) {
            const int64_t nb = std::min(chunk, batch - b0);
            ZnTransposeArgs t;
            t.src = input + b0 * plane;
            t.dst = nhwc.ptr;
            t.batch = nb;
            t.channels = c;
            t.pixels = h * w;
            const int64_t tiles = nb * cdiv(c, 32) * cdiv(h * w, 32);
            const int64_t cap = cus_now(ctx) * 16;
            if ((rc = select_device(ctx)) ||
                (rc = launch(ctx, ctx->elt[kToNhwc], (unsigned)std::min<int64_t>(tiles, cap), 1, 256, &t)) ||
                (rc = gemm_launch_ex(ctx, ZN_LAYOUT_NT, oc, hw, kdim, weights, kdim, 0, nhwc.ptr, kdim, plane,
                                     output + b0 * oc * hw, hw, oc * hw, nb, 0, bias, ZN_ACT_LINEAR, 1, &g,
                                     kGatherNhwc)))
                return rc;
        }
        return ZN_OK;
    }
    return gemm_launch_ex(ctx, ZN_LAYOUT_NN, oc, hw, kdim, weights, kdim, 0, input, hw, plane, output, hw,
                          oc * hw, batch, 0, bias, ZN_ACT_LINEAR, 1, &g);
}

int zn_hip_conv2d_forward_im2col(zn_ctx *ctx, const float *input, const float *weights, const float *bias,
                                 float *output, int64_t batch, int64_t in_channels, int64_t out_channels, int64_t k_h,
                                 int64_t k_w, int64_t in_h, int64_t in_w, int64_t out_h, int64_t out_w,
                                 int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w) {
    return conv2d_device(ctx, input, weights, bias, output, batch, in_channels, out_channels, k_h, k_w, in_h, in_w,
                         out_h, out_w, stride_h, stride_w, pad_h, pad_w, 0);
}

int zn_hip_conv2d_forward_direct(zn_ctx *ctx, const float *input, const float *weights, const float *bias,
                                 float *output, int64_t batch, int64_t in_channels, int64_t out_channels, int64_t k_h,
                                 int64_t k_w, int64_t in_h, int64_t in_w, int64_t out_h, int64_t out_w,
                                 int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w) {
    return conv2d_device(ctx, input, weights, bias, output, batch, in_channels, out_channels, k_h, k_w, in_h, in_w,
                         out_h, out_w, stride_h, stride_w, pad_h, pad_w, 1);
}

// ------------------------------------------------------- Dense backward
// One unsplit 64x64-tile GEMM of a grouped launch.
static ZnGemmArgs grouped_gemm_args(const float *a, int64_t lda, const float *b, int64_t ldb, float *c, int64_t ldc,
                                    int64_t m, int64_t n, int64_t k, int tile = 64) {
    ZnGemmArgs g;
    std::memset(&g, 0, sizeof(g));
    g.a = a;
    g.b = b;
    g.c = c;
    g.lda = lda;
    g.ldb = ldb;
    g.ldc = ldc;
    g.m = (int32_t)m;
    g.n = (int32_t)n;
    g.k = (int32_t)k;
    g.tiles_m = (int32_t)cdiv(m, tile);
    g.tiles_n = (int32_t)cdiv(n, tile);
    g.act = ZN_ACT_LINEAR;
    g.vec_c = aligned16(c) && ldc % 4 == 0;
    g.group_m = 1;
    g.splits = 1;
    g.k_chunk = (int32_t)k;
    return g;
}

// zn_dense_bwd_m[_v]: grad_input = gaa . W^T (NT, skipped when null),
// grad_weights = input^T . gaa (TN) and the bias gradient in one launch: the
// ordered sum of a prologue's partials (r, bias_blocks workgroups), or, with
// cs.splits > 0, the column sums of gaa themselves (cs).
// tile 32: zn_dense_bwd_k[_v], the same on 32x32 tiles whose four waves split
// K; only these tiles can also write the layer below's grad_after_act
// (chain_*) as they finish grad_input.
static int dense_backward_grouped(zn_ctx *ctx, const float *input, const float *weights, const float *gaa,
                                  float *grad_input, float *grad_weights, const ZnReduceArgs &r, int bias_blocks,
                                  const ZnColSumArgs &cs, int64_t batch, int64_t in_size, int64_t out_size, int wg_nt,
                                  int wg_tn, int tile, int chain_act, const float *chain_y, float *chain_gaa) {
    ZnDenseBwdArgs d;
    std::memset(&d, 0, sizeof(d));
    if (grad_input) {
        d.nt = grouped_gemm_args(gaa, out_size, weights, out_size, grad_input, in_size, batch, in_size, out_size, tile);
        d.nt.chain_y = chain_y;
        d.nt.chain_gaa = chain_gaa;
        d.nt.chain_act = chain_act;
    }
    d.tn = grouped_gemm_args(input, in_size, gaa, out_size, grad_weights, out_size, in_size, out_size, batch, tile);
    d.wg_nt = wg_nt;
    d.wg_tn = wg_tn;
    if (cs.splits > 0) {
        d.colsum = cs;
        d.wg_colsum = (int32_t)cdiv(out_size, 16);
    } else {
        d.bias = r;
        d.wg_bias = bias_blocks;
    }
    // 16-byte staging when every staged row is a whole number of aligned float4s
    const bool vec_tn = aligned16(input) && aligned16(gaa) && in_size % 4 == 0 && out_size % 4 == 0;
    const bool vec_nt = !grad_input || (aligned16(weights) && out_size % 4 == 0);
    hipFunction_t f = (tile == 32 ? ctx->dense_bwd_k : ctx->dense_bwd)[vec_tn && vec_nt ? 1 : 0];
    return launch(ctx, f, (unsigned)(wg_nt + wg_tn + (cs.splits > 0 ? d.wg_colsum : bias_blocks)), 1, 256, &d);
}

// Dense.backward (src/layer.zig:411-475) on device pointers:
//   gaa = activationBackward(act, y, grad_output)  and  grad_bias += sum_rows gaa
// in one pass (zn_dense_grad_prologue: per-split column sums, then the
// split-K reduce adds the splits in ascending order onto grad_bias), then
// grad_input = gaa . W^T (NT) and grad_weights = input^T . gaa (TN,
// overwritten like the reference).  grad_input may be null (first layer).
//
// Chaining (zn_hip_dense_backward_chain): with gaa_ready, grad_after_act
// already holds this layer's gaa (y and grad_output are not read) and only
// its column sums are taken; with prev_gaa, the layer below's
// prev_gaa = activationBackward(prev_act, prev_y, grad_input) is written too.
// A linear layer's gaa is grad_output itself, so it needs no prologue either:
// the GEMMs read grad_output and the column-sum workgroups copy it into
// grad_after_act.  Every sum keeps the unchained order (the same row splits,
// rows ascending within a split, splits ascending), so both ways give the
// same bits.
static int dense_backward_impl(zn_ctx *ctx, int act, const float *input, const float *weights,
                               const float *activated_output, const float *grad_output, float *grad_after_act,
                               float *grad_input, float *grad_weights, float *grad_bias, int64_t batch,
                               int64_t in_size, int64_t out_size, bool gaa_ready, int prev_act, const float *prev_y,
                               float *prev_gaa) {
    if (!ctx || act < ZN_ACT_LINEAR || act > ZN_ACT_TANH || batch < 0 || in_size < 0 || out_size < 0)
        return ZN_ERR_INVALID_ARG;
    if (prev_gaa && (prev_act < ZN_ACT_LINEAR || prev_act > ZN_ACT_TANH)) return ZN_ERR_INVALID_ARG;
    if (batch > INT_MAX || in_size > INT_MAX || out_size > INT_MAX) return ZN_ERR_OVERFLOW;
    if (out_size == 0) return ZN_OK;
    if (batch > 0 && (!grad_after_act || !grad_bias || (!gaa_ready && (!activated_output || !grad_output))))
        return ZN_ERR_INVALID_ARG;
    if (in_size > 0 && (!grad_weights || (batch > 0 && (!input || !weights)))) return ZN_ERR_INVALID_ARG;
    if (prev_gaa && batch > 0 && in_size > 0 && (!grad_input || !prev_y)) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    const bool chain = prev_gaa && batch > 0 && in_size > 0;
    if (batch > 0) {
        const int64_t cus = cus_now(ctx);
        const int64_t col_groups = cdiv(out_size, 256);
        // enough row splits for ~4 workgroups per CU, at least 16 rows each
        int64_t splits = std::max<int64_t>(1, std::min<int64_t>(cdiv(batch, 16), 4 * cus / col_groups));
        if (splits > 65535) splits = 65535;
        const int64_t per = cdiv(batch, splits);
        splits = cdiv(batch, per);
        // gaa without a prologue: a ready buffer, or grad_output of a linear layer
        const bool no_prologue = gaa_ready || act == ZN_ACT_LINEAR;
        const float *gaa = gaa_ready ? grad_after_act : (act == ZN_ACT_LINEAR ? grad_output : grad_after_act);
        // Small layers: grad_input, grad_weights and the bias gradient in one
        // launch (C2's layers: 5 launches -> 2, or 1 without a prologue).  Up
        // to 2 workgroups per CU of 32x32 tiles whose four waves split K (C2
        // step 44 -> 33 us), else up to 2 per CU of unsplit 64x64 tiles.
        const bool small = in_size > 0 && batch <= 2048 && out_size <= 2048 && ctx->forced_tile < 0 &&
                           ctx->forced_splits == 0 && in_size <= INT_MAX / 4 / std::max<int64_t>(batch, out_size);
        int tile = 0;
        int64_t wg_nt = 0, wg_tn = 0;
        for (int t : {32, 64}) {
            wg_nt = grad_input ? cdiv(batch, t) * cdiv(in_size, t) : 0;
            wg_tn = cdiv(in_size, t) * cdiv(out_size, t);
            if (t == 32 && ctx->forced_wave_split == 0) continue;
            if (small && wg_nt + wg_tn <= 2 * cus) {
                tile = t;
                break;
            }
        }
        ZnColSumArgs cs;
        std::memset(&cs, 0, sizeof(cs));
        if (tile && no_prologue && splits <= kMaxColSumSplits) {
            // one launch: the column sums run beside the GEMMs
            cs.src = gaa;
            cs.dst = grad_bias;
            cs.copy = gaa_ready ? nullptr : grad_after_act;
            cs.rows = (int32_t)batch;
            cs.n = (int32_t)out_size;
            cs.per = (int32_t)per;
            cs.splits = (int32_t)splits;
            ZnReduceArgs none;
            std::memset(&none, 0, sizeof(none));
            const bool fused_chain = chain && tile == 32;
            if ((rc = dense_backward_grouped(ctx, input, weights, gaa, grad_input, grad_weights, none, 0, cs, batch,
                                             in_size, out_size, (int)wg_nt, (int)wg_tn, tile, prev_act,
                                             fused_chain ? prev_y : nullptr, fused_chain ? prev_gaa : nullptr)))
                return rc;
            if (chain && !fused_chain)
                return zn_hip_activation_backward(ctx, prev_act, prev_y, grad_input, prev_gaa, batch * in_size);
            return ZN_OK;
        }
        Lease part(ctx);
        if ((rc = part.get((size_t)(splits * out_size)))) return rc;
        ZnDenseGradArgs g;
        if (gaa_ready) {  // the sums only: gaa read as the grad_output of a linear activation
            g.y = grad_after_act;
            g.go = grad_after_act;
            g.gaa = nullptr;
            g.act = ZN_ACT_LINEAR;
        } else {
            g.y = activated_output;
            g.go = grad_output;
            g.gaa = grad_after_act;
            g.act = act;
        }
        g.partial = part.ptr;
        g.rows = batch;
        g.n = out_size;
        g.rows_per_split = (int32_t)per;
        if ((rc = launch(ctx, ctx->elt[kDenseGrad], (unsigned)col_groups, (unsigned)splits, 256, &g))) return rc;
        ZnReduceArgs r;
        std::memset(&r, 0, sizeof(r));
        r.ws = part.ptr;
        r.c = grad_bias;
        r.m = 1;
        r.n = (int32_t)out_size;
        r.ldc = out_size;
        r.batch = 1;
        r.splits = (int32_t)splits;
        r.accumulate = 1;
        r.act = ZN_ACT_LINEAR;
        r.vec = (out_size % 4 == 0 && aligned16(grad_bias) && aligned16(part.ptr)) ? 1 : 0;
        const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(cdiv(out_size / (r.vec ? 4 : 1), 256), 8 * cus));
        if (tile) {
            const bool fused_chain = chain && tile == 32;
            if ((rc = dense_backward_grouped(ctx, input, weights, grad_after_act, grad_input, grad_weights, r,
                                             (int)blocks, cs, batch, in_size, out_size, (int)wg_nt, (int)wg_tn, tile,
                                             prev_act, fused_chain ? prev_y : nullptr,
                                             fused_chain ? prev_gaa : nullptr)))
                return rc;
            if (chain && !fused_chain)
                return zn_hip_activation_backward(ctx, prev_act, prev_y, grad_input, prev_gaa, batch * in_size);
            return ZN_OK;
        }
        if ((rc = launch(ctx, ctx->splitk_reduce, (unsigned)blocks, 1, 256, &r))) return rc;
    }
    if (in_size == 0) return ZN_OK;
    if (grad_input && batch > 0 &&
        (rc = gemm_launch(ctx, ZN_LAYOUT_NT, batch, in_size, out_size, grad_after_act, out_size, 0, weights, out_size,
                          0, grad_input, in_size, 0, 1, 0, nullptr, ZN_ACT_LINEAR)))
        return rc;
    if (chain && (rc = zn_hip_activation_backward(ctx, prev_act, prev_y, grad_input, prev_gaa, batch * in_size)))
        return rc;
    if (batch == 0) return zn_hip_fill_f32(ctx, grad_weights, 0.0f, in_size * out_size);
    return gemm_launch(ctx, ZN_LAYOUT_TN, in_size, out_size, batch, input, in_size, 0, grad_after_act, out_size, 0,
                       grad_weights, out_size, 0, 1, 0, nullptr, ZN_ACT_LINEAR);
}

int zn_hip_dense_backward(zn_ctx *ctx, int act, const float *input, const float *weights,
                          const float *activated_output, const float *grad_output, float *grad_after_act,
                          float *grad_input, float *grad_weights, float *grad_bias, int64_t batch, int64_t in_size,
                          int64_t out_size) {
    return dense_backward_impl(ctx, act, input, weights, activated_output, grad_output, grad_after_act, grad_input,
                               grad_weights, grad_bias, batch, in_size, out_size, false, ZN_ACT_LINEAR, nullptr,
                               nullptr);
}

int zn_hip_dense_backward_chain(zn_ctx *ctx, int act, const float *input, const float *weights,
                                const float *activated_output, const float *grad_output, float *grad_after_act,
                                float *grad_input, float *grad_weights, float *grad_bias, int64_t batch,
                                int64_t in_size, int64_t out_size, int gaa_ready, int prev_act,
                                const float *prev_activated_output, float *prev_grad_after_act) {
    if (gaa_ready != 0 && gaa_ready != 1) return ZN_ERR_INVALID_ARG;
    return dense_backward_impl(ctx, act, input, weights, activated_output, grad_output, grad_after_act, grad_input,
                               grad_weights, grad_bias, batch, in_size, out_size, gaa_ready == 1, prev_act,
                               prev_activated_output, prev_grad_after_act);
}

// ------------------------------------------------- two stacked Dense layers
// The pair kernels (kernels/mlp_f32.hip) take a top layer of at most 16
// outputs.
constexpr int64_t kPairOutMax = 16;
// The backward's LDS copies of W2 (all rows, padded to 32) and of gaa2 (all
// rows, padded to 32), read 16 bytes at a time.
constexpr int64_t kPairRawW = 2048, kPairRawG = 4096;

static ZnPairGemm pair_gemm(const float *src, int64_t ld, float *c, int64_t ldc, int64_t m, int64_t n, int64_t k) {
    ZnPairGemm g;
    g.src = src;
    g.c = c;
    g.ld = (int32_t)ld;
    g.ldc = (int32_t)ldc;
    g.m = (int32_t)m;
    g.n = (int32_t)n;
    g.k = (int32_t)k;
    g.tiles_n = (int32_t)cdiv(n, 32);
    return g;
}

// The path tests force (a tile, a split or no wave split) takes the
// per-layer launches.
static bool pair_forced_off(const zn_ctx *ctx) {
    return ctx->forced_tile >= 0 || ctx->forced_splits != 0 || ctx->forced_wave_split == 0;
}

static bool pair_extents_ok(int64_t batch, int64_t in_size, int64_t hidden, int64_t out_size) {
    const int64_t lim = (int64_t)INT_MAX / 4;
    return batch * in_size <= lim && in_size * hidden <= lim && batch * hidden <= lim &&
           hidden * out_size <= lim && batch * out_size <= lim;
}

// Network.forward over two Dense layers (src/network.zig:309-360, which runs
// Dense.forward, src/layer.zig:380-409, per layer): h = act1(x . W1 + b1),
// then y = act2(h . W2 + b2).  One launch (zn_dense_pair_fwd) when the top
// layer has at most 16 outputs and the lower layer's 16x16 tiles are at most
// one per CU; otherwise the two fused GEMMs of Backend.matMulBias*.
int zn_hip_dense_pair_forward(zn_ctx *ctx, int act1, const float *x, const float *w1, const float *b1, float *h,
                              int act2, const float *w2, const float *b2, float *y, int64_t batch, int64_t in_size,
                              int64_t hidden, int64_t out_size) {
    if (!ctx || act1 < ZN_ACT_LINEAR || act1 > ZN_ACT_TANH || act2 < ZN_ACT_LINEAR || act2 > ZN_ACT_TANH ||
        batch < 0 || in_size < 0 || hidden < 0 || out_size < 0)
        return ZN_ERR_INVALID_ARG;
    // a Dense layer has at least one input and one output (Dense.init, src/layer.zig:304-305)
    if (in_size == 0 || hidden == 0 || out_size == 0) return ZN_ERR_INVALID_ARG;
    if (batch > INT_MAX || in_size > INT_MAX || hidden > INT_MAX || out_size > INT_MAX) return ZN_ERR_OVERFLOW;
    if (batch == 0) return ZN_OK;
    if (!x || !w1 || !h || !w2 || !y) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    const int64_t tiles_m = cdiv(batch, 16), tiles_n = cdiv(hidden, 16);
    // the tiles' partial sums of y go to the workspace (256 floats per tile)
    const size_t part_bytes = (size_t)(tiles_m * tiles_n) * 256 * sizeof(float);
    const bool fused = out_size <= kPairOutMax && tiles_m * tiles_n <= cus_now(ctx) && tiles_m <= kCounterSlots &&
                       !pair_forced_off(ctx) && pair_extents_ok(batch, in_size, hidden, out_size) && !ctx->no_alloc &&
                       ensure_workspace(ctx, part_bytes) == ZN_OK;
    if (!fused) {
        if ((rc = gemm_launch(ctx, ZN_LAYOUT_NN, batch, hidden, in_size, x, in_size, 0, w1, hidden, 0, h, hidden, 0,
                              1, 0, b1, act1)))
            return rc;
        return gemm_launch(ctx, ZN_LAYOUT_NN, batch, out_size, hidden, h, hidden, 0, w2, out_size, 0, y, out_size, 0,
                           1, 0, b2, act2);
    }
    ZnPairFwdArgs a;
    std::memset(&a, 0, sizeof(a));
    ZnGemmArgs &p = a.l1;
    p.a = x;
    p.b = w1;
    p.c = h;
    p.bias = b1;
    p.lda = in_size;
    p.ldb = hidden;
    p.ldc = hidden;
    p.m = (int32_t)batch;
    p.n = (int32_t)hidden;
    p.k = (int32_t)in_size;
    p.tiles_m = (int32_t)tiles_m;
    p.tiles_n = (int32_t)tiles_n;
    p.act = act1;
    p.group_m = 1;
    p.splits = 1;
    p.k_chunk = (int32_t)in_size;
    p.batch = 1;
    a.w2 = w2;
    a.b2 = b2;
    a.y = y;
    a.part = ctx->ws;
    a.counters = ctx->counters;
    a.out = (int32_t)out_size;
    a.act2 = act2;
    const bool vec = aligned16(x) && aligned16(w1) && in_size % 4 == 0 && hidden % 4 == 0;
    return launch(ctx, ctx->pair_fwd[vec ? 1 : 0], (unsigned)(tiles_m * tiles_n), 1,
                  (unsigned)ctx->pair_fwd_threads[vec ? 1 : 0], &a);
}

// The backward loop of Network over the same two layers (src/network.zig:
// 455-477: Dense.backward per layer, top first, src/layer.zig:411-475):
//   gaa2 = act2'(y, grad_y), grad_h = gaa2 . W2^T, grad_w2 = h^T . gaa2,
//   grad_b2 += column sums of gaa2;
//   gaa1 = act1'(h, grad_h), grad_x = gaa1 . W1^T (skipped when null),
//   grad_w1 = x^T . gaa1, grad_b1 += column sums of gaa1.
// One launch (zn_dense_pair_bwd) when the top layer has at most 16 outputs
// and the workgroups fit two per CU; otherwise the chained per-layer
// launches of zn_hip_dense_backward_chain.
int zn_hip_dense_pair_backward(zn_ctx *ctx, int act1, const float *x, const float *w1, const float *h, float *gaa1,
                               float *grad_x, float *grad_w1, float *grad_b1, int act2, const float *w2,
                               const float *y, const float *grad_y, float *gaa2, float *grad_h, float *grad_w2,
                               float *grad_b2, int64_t batch, int64_t in_size, int64_t hidden, int64_t out_size) {
    if (!ctx || act1 < ZN_ACT_LINEAR || act1 > ZN_ACT_TANH || act2 < ZN_ACT_LINEAR || act2 > ZN_ACT_TANH ||
        batch < 0 || in_size < 0 || hidden < 0 || out_size < 0)
        return ZN_ERR_INVALID_ARG;
    if (in_size == 0 || hidden == 0 || out_size == 0) return ZN_ERR_INVALID_ARG;  // Dense.init, src/layer.zig:304-305
    if (batch > INT_MAX || in_size > INT_MAX || hidden > INT_MAX || out_size > INT_MAX) return ZN_ERR_OVERFLOW;
    if (batch > 0 && (!gaa2 || !grad_b2 || !grad_y || (act2 != ZN_ACT_LINEAR && !y) || !grad_h || !w2 || !h ||
                      !gaa1 || !grad_b1 || !x || !w1))
        return ZN_ERR_INVALID_ARG;
    if (!grad_w2 || !grad_w1) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    const int64_t wg_nt = grad_x ? cdiv(batch, 32) * cdiv(in_size, 64) : 0;
    const int64_t wg_tn1 = cdiv(in_size, 32) * cdiv(hidden, 32);
    const int64_t wg_tn2 = cdiv(hidden, 32);
    // one workgroup per CU (107 KB of LDS each), all resident at once
    const bool fused = batch >= 1 && out_size <= kPairOutMax && wg_nt + wg_tn1 + wg_tn2 <= cus_now(ctx) &&
                       !pair_forced_off(ctx) &&
                       pair_extents_ok(batch, in_size, hidden, out_size) &&
                       cdiv(hidden, 32) * 32 * out_size <= kPairRawW && cdiv(batch, 32) * 32 * out_size <= kPairRawG &&
                       aligned16(w2) && aligned16(grad_y) && (act2 == ZN_ACT_LINEAR || aligned16(y));
    if (!fused) {
        if ((rc = dense_backward_impl(ctx, act2, h, w2, y, grad_y, gaa2, grad_h, grad_w2, grad_b2, batch, hidden,
                                      out_size, false, act1, h, gaa1)))
            return rc;
        return dense_backward_impl(ctx, act1, x, w1, nullptr, nullptr, gaa1, grad_x, grad_w1, grad_b1, batch, in_size,
                                   hidden, true, ZN_ACT_LINEAR, nullptr, nullptr);
    }
    ZnPairBwdArgs a;
    std::memset(&a, 0, sizeof(a));
    if (grad_x) {
        a.nt = pair_gemm(w1, hidden, grad_x, in_size, batch, in_size, hidden);
        a.nt.tiles_n = (int32_t)cdiv(in_size, 64);
    }
    a.tn1 = pair_gemm(x, in_size, grad_w1, hidden, in_size, hidden, batch);
    a.tn2 = pair_gemm(h, hidden, grad_w2, out_size, hidden, out_size, batch);
    a.h = h;
    a.w2 = w2;
    a.y = y;
    a.grad_y = grad_y;
    a.gaa1 = gaa1;
    a.grad_h = grad_h;
    a.gaa2 = gaa2;
    a.grad_b1 = grad_b1;
    a.grad_b2 = grad_b2;
    a.batch = (int32_t)batch;
    a.hidden = (int32_t)hidden;
    a.out = (int32_t)out_size;
    a.act1 = act1;
    a.act2 = act2;
    a.wg_nt = (int32_t)wg_nt;
    a.wg_tn1 = (int32_t)wg_tn1;
    a.wg_tn2 = (int32_t)wg_tn2;
    // 16-byte staging of the loaded operands (W1, x and h): aligned rows that are whole float4s
    const bool vec = aligned16(w1) && aligned16(x) && aligned16(h) && in_size % 4 == 0 && hidden % 4 == 0;
    return launch(ctx, ctx->pair_bwd[act1][act2 != ZN_ACT_LINEAR ? 1 : 0][vec ? 1 : 0],
                  (unsigned)(wg_nt + wg_tn1 + wg_tn2), 1, 256, &a);
}

// ------------------------------------------------------- conv backward
// Convolution backward on device.  k_order 0 follows cpuConv2dBackwardIm2col
// (src/backend.zig:3954-4065): grad_output is read as [batch*OH*OW][OC] by
// both GEMMs (grad_W = go2^T . col as one TN GEMM over all images, grad_col =
// go2 . W as an NN GEMM), W in the col K order.  k_order 1 is the direct
// branch (src/backend.zig:3064-3094), NCHW grad_output and OIHW weights:
// grad_W = sum over images of go_b . col_b (a strided-batched NN GEMM whose
// per-image products are added in image order), grad_col_b = go_b^T . W
// (strided-batched TN).  Both finish with col2im into grad_input and the
// per-channel sum of the NCHW grad_output into grad_bias.  Images are taken
// in chunks whose col buffer stays under 1 GiB.
//
// In the k_order 0 reading two of those steps become implicit GEMMs:
//  * stride_w 1, OW % 4 == 0: grad_W gathers col from the input (no im2col);
//  * stride 1, OC % 4 == 0, 16-byte-aligned grad_output: grad_input is one
//    transposed-convolution GEMM over all images (no grad_col, no col2im).
// With both, no col buffer is allocated.
static int conv2d_backward_device(zn_ctx *ctx, const float *input, const float *weights, const float *grad_output,
                                  float *grad_input, float *grad_weights, float *grad_bias, int64_t batch, int64_t c,
                                  int64_t oc, int64_t kh, int64_t kw, int64_t h, int64_t w, int64_t oh, int64_t ow,
                                  int64_t sh, int64_t sw, int64_t ph, int64_t pw, int k_order) {
    if (!ctx || !conv_dims_ok(batch, c, oc, kh, kw, h, w, oh, ow, sh, sw, ph, pw)) return ZN_ERR_INVALID_ARG;
    if (batch == 0) return ZN_OK;
    if (!input || !weights || !grad_output || !grad_input || !grad_weights || !grad_bias) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    const int64_t hw = oh * ow, taps = c * kh * kw, plane = c * h * w;
    if (hw == 0) {  // no output pixels: every gradient is zero
        if ((rc = zn_hip_fill_f32(ctx, grad_input, 0.0f, batch * plane)) ||
            (rc = zn_hip_fill_f32(ctx, grad_weights, 0.0f, oc * taps)))
            return rc;
        return zn_hip_fill_f32(ctx, grad_bias, 0.0f, oc);
    }
    const int64_t kOffsetFloats = INT_MAX / 4;  // 32-bit byte offsets per operand
    // grad_W without im2col: from an NHWC copy of the input (C % 4 == 0, any
    // stride), else by the 4-pixel gather of the NCHW input (stride_w 1,
    // OW % 4 == 0)
    const bool nhwc_w = k_order == 0 && c % 4 == 0 && plane <= kOffsetFloats && hw * oc <= kOffsetFloats;
    const bool implicit_w = k_order == 0 && (nhwc_w || (sw == 1 && ow % 4 == 0)) && plane <= kOffsetFloats &&
                            hw * oc <= kOffsetFloats;
    const bool transposed = k_order == 0 && sh == 1 && sw == 1 && oc % 4 == 0 && aligned16(grad_output) &&
                            oc * hw <= kOffsetFloats && h * w <= INT_MAX && kh * kw * oc <= INT_MAX;
    const bool need_col = !(implicit_w && transposed);
    constexpr int64_t kColFloats = (int64_t)1 << 28;  // 1 GiB of col per chunk
    int64_t chunk = batch;
    if (need_col) {
        if (hw * taps > kColFloats) return ZN_ERR_OVERFLOW;
        chunk = std::min<int64_t>(chunk, kColFloats / (hw * taps));
    }
    if (implicit_w) chunk = std::min<int64_t>(chunk, std::min(kOffsetFloats / plane, kOffsetFloats / (hw * oc)));
    Lease col(ctx), part(ctx), wt(ctx), nhwc(ctx);
    if (need_col && (rc = col.get((size_t)(chunk * hw * taps)))) return rc;
    if (nhwc_w && (rc = nhwc.get((size_t)(chunk * plane)))) return rc;
    if (k_order == 1 && (rc = part.get((size_t)(chunk * oc * taps)))) return rc;
    ZnConvGeom gw = {};  // the implicit weight gradient's gather
    if (implicit_w) {
        gw.channels = (int32_t)c;
        gw.in_h = (int32_t)h;
        gw.in_w = (int32_t)w;
        gw.k_h = (int32_t)kh;
        gw.k_w = (int32_t)kw;
        gw.out_w = (int32_t)ow;
        gw.out_h = (int32_t)oh;
        gw.stride_h = (int32_t)sh;
        gw.stride_w = (int32_t)sw;
        gw.pad_h = (int32_t)ph;
        gw.pad_w = (int32_t)pw;
        gw.k_order = 0;
        gw.div1 = (int32_t)c;
        udiv_magic((uint32_t)gw.div1, gw.div1_mul, gw.div1_shift);
        udiv_magic((uint32_t)gw.k_w, gw.kw_mul, gw.kw_shift);
        udiv_magic((uint32_t)gw.out_w, gw.ow_mul, gw.ow_shift);
        udiv_magic((uint32_t)gw.out_h, gw.oh_mul, gw.oh_shift);
    }
    for (int64_t b0 = 0; b0 < batch; b0 += chunk) {
        const int64_t nb = std::min(chunk, batch - b0);
        const int64_t rows = nb * hw;
        const float *go = grad_output + b0 * oc * hw;
        float *gi = grad_input + b0 * plane;
        if (nhwc_w) {
            // grad_W (+)= go2^T . col with col gathered from an NHWC copy of this chunk's images
            gw.images = (int32_t)nb;
            ZnTransposeArgs t;
            t.src = input + b0 * plane;
            t.dst = nhwc.ptr;
            t.batch = nb;
            t.channels = c;
            t.pixels = h * w;
            const int64_t tiles = nb * cdiv(c, 32) * cdiv(h * w, 32);
            const int64_t cap = cus_now(ctx) * 16;
            if ((rc = launch(ctx, ctx->elt[kToNhwc], (unsigned)std::min<int64_t>(tiles, cap), 1, 256, &t)) ||
                (rc = gemm_launch_ex(ctx, ZN_LAYOUT_TN, oc, taps, rows, go, oc, 0, nhwc.ptr, taps, 0, grad_weights,
                                     taps, 0, 1, b0 > 0, nullptr, ZN_ACT_LINEAR, 0, &gw, kGatherWeightNhwc)))
                return rc;
        } else if (implicit_w) {
            // grad_W (+)= go2^T . col with col gathered from this chunk's images: TN, M = OC, N = taps, K = rows
            gw.images = (int32_t)nb;
            if ((rc = gemm_launch_ex(ctx, ZN_LAYOUT_TN, oc, taps, rows, go, oc, 0, input + b0 * plane, taps, 0,
                                     grad_weights, taps, 0, 1, b0 > 0, nullptr, ZN_ACT_LINEAR, 0, &gw,
                                     kGatherWeightGrad)))
                return rc;
        } else {
            ZnIm2colArgs ia = col_args(const_cast<float *>(input) + b0 * plane, col.ptr, nb, c, kh, kw, h, w, oh, ow,
                                       sh, sw, ph, pw, k_order);
            if ((rc = im2col_launch(ctx, ia))) return rc;
        }
        if (k_order == 0) {
            // grad_W (+)= go2^T . col: TN, M = OC, N = taps, K = rows
            if (!implicit_w && (rc = gemm_launch(ctx, ZN_LAYOUT_TN, oc, taps, rows, go, oc, 0, col.ptr, taps, 0,
                                                 grad_weights, taps, 0, 1, b0 > 0, nullptr, ZN_ACT_LINEAR)))
                return rc;
            if (transposed) continue;  // grad_input after the loop
            // grad_col = go2 . W: NN, M = rows, N = taps, K = OC (into the col buffer)
            if ((rc = gemm_launch(ctx, ZN_LAYOUT_NN, rows, taps, oc, go, oc, 0, weights, taps, 0, col.ptr, taps, 0, 1,
                                  0, nullptr, ZN_ACT_LINEAR)))
                return rc;
        } else {
            // per image go_b [OC x HW] . col_b [HW x taps] -> part[b], then summed in image order
            if ((rc = gemm_launch(ctx, ZN_LAYOUT_NN, oc, taps, hw, go, hw, oc * hw, col.ptr, taps, hw * taps, part.ptr,
                                  taps, oc * taps, nb, 0, nullptr, ZN_ACT_LINEAR)))
                return rc;
            ZnReduceArgs r;
            std::memset(&r, 0, sizeof(r));
            r.ws = part.ptr;
            r.c = grad_weights;
            r.ldc = taps;
            r.m = (int32_t)oc;
            r.n = (int32_t)taps;
            r.batch = 1;
            r.splits = (int32_t)nb;
            r.accumulate = b0 > 0;
            r.act = ZN_ACT_LINEAR;
            r.vec = (taps % 4 == 0 && aligned16(grad_weights) && aligned16(part.ptr)) ? 1 : 0;
            int64_t blocks = cdiv(oc * taps / (r.vec ? 4 : 1), 256);
            const int64_t cap = cus_now(ctx) * 8;
            if (blocks > cap) blocks = cap;
            if ((rc = launch(ctx, ctx->splitk_reduce, (unsigned)blocks, 1, 256, &r))) return rc;
            // grad_col_b = go_b^T . W: TN, M = HW, N = taps, K = OC, per image
            if ((rc = gemm_launch(ctx, ZN_LAYOUT_TN, hw, taps, oc, go, hw, oc * hw, weights, taps, 0, col.ptr, taps,
                                  hw * taps, nb, 0, nullptr, ZN_ACT_LINEAR)))
                return rc;
        }
        ZnIm2colArgs ca = col_args(gi, col.ptr, nb, c, kh, kw, h, w, oh, ow, sh, sw, ph, pw, k_order);
        if ((rc = col2im_launch(ctx, ca))) return rc;
    }
    if (transposed) {
        // grad_input_b[ic][(ih, iw)] = sum over (kh, kw, oc) of W'[ic][(kh*kW + kw)*OC + oc] .
        // go2[b*OH*OW + (ih + ph - kh)*OW + (iw + pw - kw)][oc]  (terms outside the output image are 0)
        const int64_t kt = kh * kw * oc;
        if ((rc = wt.get((size_t)(c * kt)))) return rc;
        ZnRegroupArgs ra;
        ra.in = weights;
        ra.out = wt.ptr;
        ra.out_channels = (int32_t)oc;
        ra.channels = (int32_t)c;
        ra.taps_per_channel = (int32_t)(kh * kw);
        const int64_t cap = cus_now(ctx) * 8;
        if ((rc = launch(ctx, ctx->elt[kRegroup], (unsigned)std::min<int64_t>(cdiv(c * kt, 256), cap), 1, 256, &ra)))
            return rc;
        ZnConvGeom g;
        std::memset(&g, 0, sizeof(g));
        g.channels = (int32_t)oc;  // gathered image: OH x OW rows of OC channels
        g.in_h = (int32_t)oh;
        g.in_w = (int32_t)ow;
        g.k_h = (int32_t)kh;
        g.k_w = (int32_t)kw;
        g.out_w = (int32_t)w;  // decodes the GEMM column into (ih, iw)
        g.stride_h = 1;
        g.stride_w = 1;
        g.pad_h = (int32_t)ph;
        g.pad_w = (int32_t)pw;
        g.div1 = (int32_t)oc;
        udiv_magic((uint32_t)g.div1, g.div1_mul, g.div1_shift);
        udiv_magic((uint32_t)g.k_w, g.kw_mul, g.kw_shift);
        udiv_magic((uint32_t)g.out_w, g.ow_mul, g.ow_shift);
        if ((rc = gemm_launch_ex(ctx, ZN_LAYOUT_NT, c, h * w, kt, wt.ptr, kt, 0, grad_output, kt, oc * hw, grad_input,
                                 h * w, plane, batch, 0, nullptr, ZN_ACT_LINEAR, 0, &g, kGatherTransposed)))
            return rc;
    }
    // grad_bias[c] = sum over images of the (image, channel) plane sums, added in image order
    Lease planes(ctx);
    if ((rc = planes.get((size_t)(batch * oc)))) return rc;
    ZnEltArgs ra;
    std::memset(&ra, 0, sizeof(ra));
    ra.out = planes.ptr;
    ra.in0 = grad_output;
    ra.rows = batch * oc;
    ra.n = hw;
    const int64_t cap = cus_now(ctx) * 16;
    if ((rc = launch(ctx, ctx->elt[kRowSum], (unsigned)std::min<int64_t>(batch * oc, cap), 1, 256, &ra))) return rc;
    if (batch > INT_MAX) return ZN_ERR_OVERFLOW;
    ZnReduceArgs r;
    std::memset(&r, 0, sizeof(r));
    r.ws = planes.ptr;
    r.c = grad_bias;
    r.m = 1;
    r.n = (int32_t)oc;
    r.ldc = oc;
    r.batch = 1;
    r.splits = (int32_t)batch;
    r.act = ZN_ACT_LINEAR;
    return launch(ctx, ctx->splitk_reduce, (unsigned)std::min<int64_t>(cdiv(oc, 256), cap), 1, 256, &r);
}

int zn_hip_col2im(zn_ctx *ctx, const float *col, float *output, int64_t batch, int64_t channels, int64_t in_h,
                  int64_t in_w, int64_t k_h, int64_t k_w, int64_t out_h, int64_t out_w, int64_t stride_h,
                  int64_t stride_w, int64_t pad_h, int64_t pad_w) {
    if (!ctx || !conv_dims_ok(batch, channels, 1, k_h, k_w, in_h, in_w, out_h, out_w, stride_h, stride_w, pad_h,
                              pad_w))
        return ZN_ERR_INVALID_ARG;
    const int64_t total = batch * channels * in_h * in_w;
    if (total == 0) return ZN_OK;
    if (!output || (!col && out_h * out_w > 0)) return ZN_ERR_INVALID_ARG;
    ZnIm2colArgs a = col_args(output, const_cast<float *>(col), batch, channels, k_h, k_w, in_h, in_w, out_h, out_w,
                              stride_h, stride_w, pad_h, pad_w, 0);
    return col2im_launch(ctx, a);
}

int zn_hip_conv2d_backward_im2col(zn_ctx *ctx, const float *input, const float *weights, const float *grad_output,
                                  float *grad_input, float *grad_weights, float *grad_bias, int64_t batch,
                                  int64_t in_channels, int64_t out_channels, int64_t k_h, int64_t k_w, int64_t in_h,
                                  int64_t in_w, int64_t out_h, int64_t out_w, int64_t stride_h, int64_t stride_w,
                                  int64_t pad_h, int64_t pad_w) {
    return conv2d_backward_device(ctx, input, weights, grad_output, grad_input, grad_weights, grad_bias, batch,
                                  in_channels, out_channels, k_h, k_w, in_h, in_w, out_h, out_w, stride_h, stride_w,
                                  pad_h, pad_w, 0);
}

int zn_hip_conv2d_backward_direct(zn_ctx *ctx, const float *input, const float *weights, const float *grad_output,
                                  float *grad_input, float *grad_weights, float *grad_bias, int64_t batch,
                                  int64_t in_channels, int64_t out_channels, int64_t k_h, int64_t k_w, int64_t in_h,
                                  int64_t in_w, int64_t out_h, int64_t out_w, int64_t stride_h, int64_t stride_w,
                                  int64_t pad_h, int64_t pad_w) {
    return conv2d_backward_device(ctx, input, weights, grad_output, grad_input, grad_weights, grad_bias, batch,
                                  in_channels, out_channels, k_h, k_w, in_h, in_w, out_h, out_w, stride_h, stride_w,
                                  pad_h, pad_w, 1);
}

int zn_hip_softmax_rows(zn_ctx *ctx, const float *in, float *out, int64_t rows, int64_t n, float scale) {
    if (!ctx || rows < 0 || n < 0) return ZN_ERR_INVALID_ARG;
    if (rows == 0 || n == 0) return ZN_OK;
    if (!in || !out) return ZN_ERR_INVALID_ARG;
    ZnEltArgs a = {};
    a.out = out;
    a.in0 = in;
    a.rows = rows;
    a.n = n;
    a.value = scale;
    int rc = select_device(ctx);
    if (rc) return rc;
    const int64_t cap = cus_now(ctx) * 8;
    return launch(ctx, ctx->elt[kSoftmax], (unsigned)(rows < cap ? rows : cap), 1, 256, &a);
}

// Per problem: S = Q.K^T (NT), P = softmax_rows(S * scale), O = P.V (NN); the
// score matrices live in a pooled buffer of batch * seq * seq floats.
// Head dims up to 128 run the fused single-pass kernel (scores never leave
// the CU); larger ones run QK^T (NT GEMM), the row softmax and P.V (NN GEMM)
// with the scores in a pooled HBM buffer.
int zn_hip_attention_forward(zn_ctx *ctx, const float *q, const float *k, const float *v, float *out, int64_t batch,
                             int64_t seq_len, int64_t d_k, float scale) {
    if (!ctx || batch < 0 || seq_len < 0 || d_k < 0) return ZN_ERR_INVALID_ARG;
    if (batch == 0 || seq_len == 0 || d_k == 0) return ZN_OK;
    if (!q || !k || !v || !out) return ZN_ERR_INVALID_ARG;
    if (seq_len > INT_MAX || d_k > INT_MAX) return ZN_ERR_OVERFLOW;
    int rc = select_device(ctx);
    if (rc) return rc;
    const int64_t sd = seq_len * d_k, ss = seq_len * seq_len;
    if (d_k <= kAttnDims[2] && sd <= (int64_t)INT_MAX / 4 && cdiv(seq_len, kAttnQueries) <= 65535) {
        const int dim = d_k <= kAttnDims[0] ? 0 : d_k <= kAttnDims[1] ? 1 : 2;
        const int vec = d_k % 4 == 0 && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out);
        ZnAttnArgs a;
        a.q = q;
        a.k = k;
        a.v = v;
        a.out = out;
        a.stride = sd;
        a.seq_len = (int32_t)seq_len;
        a.d_k = (int32_t)d_k;
        a.scale_log2 = scale * 1.44269504088896340736f;
        // grid.x = problem (so one problem's query blocks share an XCD), grid.y = query block
        const int64_t gy = cdiv(seq_len, kAttnQueries);
        constexpr int64_t kMaxGridX = (int64_t)1 << 30;
        for (int64_t b0 = 0; b0 < batch; b0 += kMaxGridX) {
            const int64_t nb = batch - b0 < kMaxGridX ? batch - b0 : kMaxGridX;
            ZnAttnArgs c = a;
            c.q = q + b0 * sd;
            c.k = k + b0 * sd;
            c.v = v + b0 * sd;
            c.out = out + b0 * sd;
            if ((rc = launch(ctx, ctx->attn[dim][vec], (unsigned)nb, (unsigned)gy, 256, &c))) return rc;
        }
        return ZN_OK;
    }
    Lease scores(ctx);
    if ((rc = scores.get((size_t)(batch * ss)))) return rc;
    if ((rc = gemm_launch(ctx, ZN_LAYOUT_NT, seq_len, seq_len, d_k, q, d_k, sd, k, d_k, sd, scores.ptr, seq_len, ss,
                          batch, 0, nullptr, ZN_ACT_LINEAR)))
        return rc;
    if ((rc = zn_hip_softmax_rows(ctx, scores.ptr, scores.ptr, batch * seq_len, seq_len, scale))) return rc;
    return gemm_launch(ctx, ZN_LAYOUT_NN, seq_len, d_k, seq_len, scores.ptr, seq_len, ss, v, d_k, sd, out, d_k, sd,
                       batch, 0, nullptr, ZN_ACT_LINEAR);
}

// ------------------------------------------------ host-slice drop-ins
int zn_hip_mat_mul(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len, float *c, size_t c_len,
                   size_t m, size_t n, size_t k, int accumulate) {
    return host_gemm(ctx, ZN_LAYOUT_NN, a, a_len, b, b_len, nullptr, 0, c, c_len, m, n, k, accumulate, ZN_ACT_LINEAR);
}

int zn_hip_mat_mul_batch(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len, float *c,
                         size_t c_len, size_t batch_size, size_t n, size_t k, int accumulate) {
    return host_gemm(ctx, ZN_LAYOUT_NN, a, a_len, b, b_len, nullptr, 0, c, c_len, batch_size, n, k, accumulate,
                     ZN_ACT_LINEAR);
}

int zn_hip_mat_mul_transpose_a(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len, float *c,
                               size_t c_len, size_t m, size_t n, size_t k, int accumulate) {
    return host_gemm(ctx, ZN_LAYOUT_TN, a, a_len, b, b_len, nullptr, 0, c, c_len, m, n, k, accumulate, ZN_ACT_LINEAR);
}

int zn_hip_mat_mul_transpose_b(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len, float *c,
                               size_t c_len, size_t m, size_t n, size_t k, int accumulate) {
    return host_gemm(ctx, ZN_LAYOUT_NT, a, a_len, b, b_len, nullptr, 0, c, c_len, m, n, k, accumulate, ZN_ACT_LINEAR);
}

static int host_bias_gemm(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len, const float *bias,
                          size_t bias_len, float *c, size_t c_len, size_t batch_size, size_t n, size_t k, int act) {
    if (!bias && n) return ZN_ERR_INVALID_ARG;
    return host_gemm(ctx, ZN_LAYOUT_NN, a, a_len, b, b_len, bias, bias_len, c, c_len, batch_size, n, k, 0, act);
}

int zn_hip_mat_mul_bias(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len, const float *bias,
                        size_t bias_len, float *c, size_t c_len, size_t batch_size, size_t n, size_t k) {
    return host_bias_gemm(ctx, a, a_len, b, b_len, bias, bias_len, c, c_len, batch_size, n, k, ZN_ACT_LINEAR);
}
int zn_hip_mat_mul_bias_relu(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len,
                             const float *bias, size_t bias_len, float *c, size_t c_len, size_t batch_size, size_t n,
                             size_t k) {
    return host_bias_gemm(ctx, a, a_len, b, b_len, bias, bias_len, c, c_len, batch_size, n, k, ZN_ACT_RELU);
}
int zn_hip_mat_mul_bias_sigmoid(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len,
                                const float *bias, size_t bias_len, float *c, size_t c_len, size_t batch_size,
                                size_t n, size_t k) {
    return host_bias_gemm(ctx, a, a_len, b, b_len, bias, bias_len, c, c_len, batch_size, n, k, ZN_ACT_SIGMOID);
}
int zn_hip_mat_mul_bias_tanh(zn_ctx *ctx, const float *a, size_t a_len, const float *b, size_t b_len,
                             const float *bias, size_t bias_len, float *c, size_t c_len, size_t batch_size, size_t n,
                             size_t k) {
    return host_bias_gemm(ctx, a, a_len, b, b_len, bias, bias_len, c, c_len, batch_size, n, k, ZN_ACT_TANH);
}

int zn_hip_add_bias_host(zn_ctx *ctx, float *out, size_t out_len, const float *bias, size_t bias_len) {
    if (!ctx || bias_len == 0) return ZN_ERR_INVALID_ARG;  // the reference divides by bias.len
    if (out_len && (!out || !bias)) return ZN_ERR_INVALID_ARG;
    const size_t rows = out_len / bias_len;
    if (rows == 0) return ZN_OK;
    const size_t used = rows * bias_len;
    if (ctx->capturing) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    if ((used + bias_len) * sizeof(float) <= kZeroCopyStreamBytes) {  // the kernel works on the pinned block
        if ((rc = ensure_staging(ctx))) return rc;
        PinnedBlock pb{ctx->pinned[0]};
        float *po = pb.take(used), *pbias = pb.take(bias_len);
        std::memcpy(po, out, used * sizeof(float));
        std::memcpy(pbias, bias, bias_len * sizeof(float));
        PinnedFence fence{ctx};
        if ((rc = zn_hip_add_bias(ctx, po, pbias, (int64_t)rows, (int64_t)bias_len))) return rc;
        ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        fence.done = true;
        std::memcpy(out, po, used * sizeof(float));
        return ZN_OK;
    }
    Lease dout(ctx), dbias(ctx);
    if ((rc = dout.get(used)) || (rc = dbias.get(bias_len))) return rc;
    if ((rc = copy_in(ctx, dout.ptr, out, used)) || (rc = copy_in(ctx, dbias.ptr, bias, bias_len))) return rc;
    if ((rc = zn_hip_add_bias(ctx, dout.ptr, dbias.ptr, (int64_t)rows, (int64_t)bias_len))) return rc;
    return copy_out_and_wait(ctx, out, dout.ptr, used);
}

int zn_hip_activation_forward_host(zn_ctx *ctx, int act, const float *in, size_t in_len, float *out, size_t out_len) {
    if (!ctx || act < ZN_ACT_LINEAR || act > ZN_ACT_TANH || out_len < in_len) return ZN_ERR_INVALID_ARG;
    if (in_len == 0) return ZN_OK;
    if (!in || !out) return ZN_ERR_INVALID_ARG;
    if (ctx->capturing) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    if (2 * in_len * sizeof(float) <= kZeroCopyStreamBytes) {  // the kernel works on the pinned block
        if ((rc = ensure_staging(ctx))) return rc;
        PinnedBlock pb{ctx->pinned[0]};
        float *pi = pb.take(in_len), *po = pb.take(in_len);
        std::memcpy(pi, in, in_len * sizeof(float));
        PinnedFence fence{ctx};
        if ((rc = zn_hip_activation_forward(ctx, act, pi, po, (int64_t)in_len))) return rc;
        ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        fence.done = true;
        std::memcpy(out, po, in_len * sizeof(float));
        return ZN_OK;
    }
    Lease din(ctx), dout(ctx);
    if ((rc = din.get(in_len)) || (rc = dout.get(in_len))) return rc;
    if ((rc = copy_in(ctx, din.ptr, in, in_len))) return rc;
    if ((rc = zn_hip_activation_forward(ctx, act, din.ptr, dout.ptr, (int64_t)in_len))) return rc;
    return copy_out_and_wait(ctx, out, dout.ptr, in_len);
}

int zn_hip_activation_backward_host(zn_ctx *ctx, int act, const float *y, size_t y_len, const float *grad_out,
                                    size_t grad_out_len, float *grad_in, size_t grad_in_len) {
    if (!ctx || act < ZN_ACT_LINEAR || act > ZN_ACT_TANH) return ZN_ERR_INVALID_ARG;
    if (y_len != grad_out_len || y_len != grad_in_len) return ZN_ERR_INVALID_ARG;
    if (y_len == 0) return ZN_OK;
    if (!y || !grad_out || !grad_in) return ZN_ERR_INVALID_ARG;
    if (ctx->capturing) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    if (3 * y_len * sizeof(float) <= kZeroCopyStreamBytes) {  // the kernel works on the pinned block
        if ((rc = ensure_staging(ctx))) return rc;
        PinnedBlock pb{ctx->pinned[0]};
        float *py = pb.take(y_len), *pgo = pb.take(y_len), *pgi = pb.take(y_len);
        std::memcpy(py, y, y_len * sizeof(float));
        std::memcpy(pgo, grad_out, y_len * sizeof(float));
        PinnedFence fence{ctx};
        if ((rc = zn_hip_activation_backward(ctx, act, py, pgo, pgi, (int64_t)y_len))) return rc;
        ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        fence.done = true;
        std::memcpy(grad_in, pgi, y_len * sizeof(float));
        return ZN_OK;
    }
    Lease dy(ctx), dgo(ctx), dgi(ctx);
    if ((rc = dy.get(y_len)) || (rc = dgo.get(y_len)) || (rc = dgi.get(y_len))) return rc;
    if ((rc = copy_in(ctx, dy.ptr, y, y_len)) || (rc = copy_in(ctx, dgo.ptr, grad_out, y_len))) return rc;
    if ((rc = zn_hip_activation_backward(ctx, act, dy.ptr, dgo.ptr, dgi.ptr, (int64_t)y_len))) return rc;
    return copy_out_and_wait(ctx, grad_in, dgi.ptr, y_len);
}

int zn_hip_accumulate_bias_host(zn_ctx *ctx, float *grad_bias, size_t grad_bias_len, const float *gaa,
                                size_t gaa_len) {
    if (!ctx || grad_bias_len == 0) return ZN_ERR_INVALID_ARG;
    if (gaa_len && (!grad_bias || !gaa)) return ZN_ERR_INVALID_ARG;
    const size_t rows = gaa_len / grad_bias_len;
    if (rows == 0) return ZN_OK;
    if (ctx->capturing) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    if ((rows + 1) * grad_bias_len * sizeof(float) <= kSmallHostBytes) {
        // gaa goes up in one DMA from the pinned block; grad_bias (one read and
        // one write per thread) stays in it
        if ((rc = ensure_staging(ctx))) return rc;
        PinnedBlock pb{ctx->pinned[0]};
        float *pgaa = pb.take(rows * grad_bias_len), *pgb = pb.take(grad_bias_len);
        std::memcpy(pgaa, gaa, rows * grad_bias_len * sizeof(float));
        std::memcpy(pgb, grad_bias, grad_bias_len * sizeof(float));
        Lease dgaa(ctx);
        PinnedFence fence{ctx};
        if ((rc = dgaa.get(rows * grad_bias_len))) return rc;
        ZN_HIP_TRY(ctx, hipMemcpyAsync(dgaa.ptr, pgaa, rows * grad_bias_len * sizeof(float), hipMemcpyHostToDevice,
                                       ctx->stream));
        if ((rc = zn_hip_accumulate_bias(ctx, pgb, dgaa.ptr, (int64_t)rows, (int64_t)grad_bias_len))) return rc;
        ZN_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        fence.done = true;
        std::memcpy(grad_bias, pgb, grad_bias_len * sizeof(float));
        return ZN_OK;
    }
    Lease dgb(ctx), dgaa(ctx);
    if ((rc = dgb.get(grad_bias_len)) || (rc = dgaa.get(rows * grad_bias_len))) return rc;
    if ((rc = copy_in(ctx, dgb.ptr, grad_bias, grad_bias_len)) || (rc = copy_in(ctx, dgaa.ptr, gaa, rows * grad_bias_len)))
        return rc;
    if ((rc = zn_hip_accumulate_bias(ctx, dgb.ptr, dgaa.ptr, (int64_t)rows, (int64_t)grad_bias_len))) return rc;
    return copy_out_and_wait(ctx, grad_bias, dgb.ptr, grad_bias_len);
}

int zn_hip_conv2d_forward_host(zn_ctx *ctx, const float *input, size_t input_len, const float *weights,
                               size_t weights_len, const float *bias, size_t bias_len, float *output,
                               size_t output_len, size_t in_channels, size_t out_channels, size_t k_h, size_t k_w,
                               size_t in_h, size_t in_w, size_t out_h, size_t out_w, size_t stride_h, size_t stride_w,
                               size_t pad_h, size_t pad_w) {
    if (!ctx || in_channels == 0 || in_h == 0 || in_w == 0) return ZN_ERR_INVALID_ARG;
    const int64_t lim = INT_MAX;
    if ((int64_t)in_channels > lim || (int64_t)out_channels > lim || (int64_t)k_h > lim || (int64_t)k_w > lim ||
        (int64_t)in_h > lim || (int64_t)in_w > lim || (int64_t)out_h > lim || (int64_t)out_w > lim)
        return ZN_ERR_OVERFLOW;
    const size_t plane = in_channels * in_h * in_w;
    const size_t batch = input_len / plane;  // batch_size = input.len / (C*H*W) (src/backend.zig:3005)
    const size_t kdim = in_channels * k_h * k_w;
    const size_t out_count = batch * out_channels * out_h * out_w;
    if (weights_len < out_channels * kdim || bias_len < out_channels || output_len < out_count)
        return ZN_ERR_INVALID_ARG;
    if (out_count == 0) return ZN_OK;
    if (!input || !weights || !bias || !output) return ZN_ERR_INVALID_ARG;
    // the reference's switch (src/backend.zig:3009-3016): im2col semantics for
    // large problems with kernels of 9+ taps, direct convolution otherwise
    const bool use_im2col = out_count >= 1024 && k_h * k_w >= 9;
    int rc = select_device(ctx);
    if (rc) return rc;
    Lease din(ctx), dw(ctx), db(ctx), dout(ctx);
    if ((rc = din.get(batch * plane)) || (rc = dw.get(out_channels * kdim)) || (rc = db.get(out_channels)) ||
        (rc = dout.get(out_count)))
        return rc;
    if ((rc = copy_in(ctx, din.ptr, input, batch * plane)) || (rc = copy_in(ctx, dw.ptr, weights, out_channels * kdim)) ||
        (rc = copy_in(ctx, db.ptr, bias, out_channels)))
        return rc;
    rc = conv2d_device(ctx, din.ptr, dw.ptr, db.ptr, dout.ptr, (int64_t)batch, (int64_t)in_channels,
                       (int64_t)out_channels, (int64_t)k_h, (int64_t)k_w, (int64_t)in_h, (int64_t)in_w, (int64_t)out_h,
                       (int64_t)out_w, (int64_t)stride_h, (int64_t)stride_w, (int64_t)pad_h, (int64_t)pad_w,
                       use_im2col ? 0 : 1);
    if (rc) return rc;
    return copy_out_and_wait(ctx, output, dout.ptr, out_count);
}

int zn_hip_conv2d_backward_host(zn_ctx *ctx, const float *input, size_t input_len, const float *weights,
                                size_t weights_len, const float *grad_output, size_t grad_output_len,
                                float *grad_input, size_t grad_input_len, float *grad_weights, size_t grad_weights_len,
                                float *grad_bias, size_t grad_bias_len, size_t in_channels, size_t out_channels,
                                size_t k_h, size_t k_w, size_t in_h, size_t in_w, size_t out_h, size_t out_w,
                                size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w) {
    if (!ctx || in_channels == 0 || in_h == 0 || in_w == 0) return ZN_ERR_INVALID_ARG;
    const int64_t lim = INT_MAX;
    if ((int64_t)in_channels > lim || (int64_t)out_channels > lim || (int64_t)k_h > lim || (int64_t)k_w > lim ||
        (int64_t)in_h > lim || (int64_t)in_w > lim || (int64_t)out_h > lim || (int64_t)out_w > lim)
        return ZN_ERR_OVERFLOW;
    const size_t plane = in_channels * in_h * in_w;
    const size_t batch = input_len / plane;  // batch_size = input.len / (C*H*W) (src/backend.zig:3050)
    const size_t taps = in_channels * k_h * k_w;
    const size_t out_count = batch * out_channels * out_h * out_w;
    if (weights_len < out_channels * taps || grad_output_len < out_count || grad_input_len < batch * plane ||
        grad_weights_len < out_channels * taps || grad_bias_len < out_channels)
        return ZN_ERR_INVALID_ARG;
    if (batch == 0) return ZN_OK;
    if (!input || !weights || !grad_output || !grad_input || !grad_weights || !grad_bias) return ZN_ERR_INVALID_ARG;
    // the reference's switch (src/backend.zig:3053-3062)
    const bool use_im2col = out_count >= 1024 && k_h * k_w >= 9;
    int rc = select_device(ctx);
    if (rc) return rc;
    Lease din(ctx), dw(ctx), dgo(ctx), dgi(ctx), dgw(ctx), dgb(ctx);
    if ((rc = din.get(batch * plane)) || (rc = dw.get(out_channels * taps)) || (rc = dgo.get(out_count)) ||
        (rc = dgi.get(batch * plane)) || (rc = dgw.get(out_channels * taps)) || (rc = dgb.get(out_channels)))
        return rc;
    if ((rc = copy_in(ctx, din.ptr, input, batch * plane)) || (rc = copy_in(ctx, dw.ptr, weights, out_channels * taps)) ||
        (rc = copy_in(ctx, dgo.ptr, grad_output, out_count)))
        return rc;
    rc = conv2d_backward_device(ctx, din.ptr, dw.ptr, dgo.ptr, dgi.ptr, dgw.ptr, dgb.ptr, (int64_t)batch,
                                (int64_t)in_channels, (int64_t)out_channels, (int64_t)k_h, (int64_t)k_w, (int64_t)in_h,
                                (int64_t)in_w, (int64_t)out_h, (int64_t)out_w, (int64_t)stride_h, (int64_t)stride_w,
                                (int64_t)pad_h, (int64_t)pad_w, use_im2col ? 0 : 1);
    if (rc) return rc;
    ZN_HIP_TRY(ctx, hipMemcpyAsync(grad_weights, dgw.ptr, out_channels * taps * sizeof(float), hipMemcpyDeviceToHost,
                                   ctx->stream));
    ZN_HIP_TRY(ctx, hipMemcpyAsync(grad_bias, dgb.ptr, out_channels * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
    return copy_out_and_wait(ctx, grad_input, dgi.ptr, batch * plane);
}

int zn_hip_attention_forward_host(zn_ctx *ctx, const float *q, size_t q_len, const float *k, size_t k_len,
                                  const float *v, size_t v_len, float *output, size_t output_len, float *scores,
                                  size_t scores_len, size_t seq_len, size_t d_k, float scale) {
    (void)scores;  // the device path keeps its scores in HBM
    if (!ctx) return ZN_ERR_INVALID_ARG;
    size_t sd;
    if (!mul_ok(seq_len, d_k, &sd)) return ZN_ERR_OVERFLOW;
    if (q_len < sd || k_len < sd || v_len < sd || output_len < sd || scores_len < seq_len) return ZN_ERR_INVALID_ARG;
    if (sd == 0) return ZN_OK;
    if (!q || !k || !v || !output) return ZN_ERR_INVALID_ARG;
    int rc = select_device(ctx);
    if (rc) return rc;
    Lease dq(ctx), dk(ctx), dv(ctx), dout(ctx);
    if ((rc = dq.get(sd)) || (rc = dk.get(sd)) || (rc = dv.get(sd)) || (rc = dout.get(sd))) return rc;
    if ((rc = copy_in(ctx, dq.ptr, q, sd)) || (rc = copy_in(ctx, dk.ptr, k, sd)) || (rc = copy_in(ctx, dv.ptr, v, sd)))
        return rc;
    if ((rc = zn_hip_attention_forward(ctx, dq.ptr, dk.ptr, dv.ptr, dout.ptr, 1, (int64_t)seq_len, (int64_t)d_k, scale)))
        return rc;
    return copy_out_and_wait(ctx, output, dout.ptr, sd);
}

}  // extern "C"
