//! hip.zig -- ZigNeuron's binding of the MI355X (gfx950) GEMM backend.
//!
//! Replaces, for the GEMM path, cuda.zig / cuda_driver.zig / cuda_nvrtc.zig /
//! cuda_kernels.zig: a thin `extern` layer over the C ABI of libzn_hip
//! (include/zn_hip.h), which loads offline-built gfx950 code objects, and a
//! `HipBackend` shaped like `CudaBackend` (src/cuda.zig:540, 729, 1008, 2255,
//! 2284, 3026) for the `hip_backend` dispatch added to src/backend.zig by
//! backend_hip.patch.  Every function of zn_hip.h is declared here, with the
//! same parameter names; tests/test_zig_binding.py checks this file against
//! the header (names, arity and C types).
//!
//! Conventions of the ABI: every call returns a status (0 or a negative
//! ZN_ERR_*), mapped to `HipError` by `check`; host-slice calls return when the
//! result is in host memory; device-pointer calls are ordered on the
//! context's stream.

const std = @import("std");
const activation = @import("activation.zig");

pub const Ctx = opaque {};
pub const Event = opaque {};
pub const Graph = opaque {};

/// zn_device_info
pub const DeviceInfo = extern struct {
    name: [64]u8,
    compute_units: i32,
    clock_khz: i32,
    total_mem: i64,
};

pub const ABI_VERSION: c_int = 1;

pub const Layout = enum(c_int) { nn = 0, nt = 1, tn = 2 };
pub const Act = enum(c_int) { linear = 0, relu = 1, sigmoid = 2, tanh = 3 };

// ---------------------------------------------------------------- context
pub extern fn zn_hip_abi_version() c_int;
pub extern fn zn_hip_available() c_int;
pub extern fn zn_hip_create(device: c_int, code_object_dir: ?[*:0]const u8, out: *?*Ctx) c_int;
pub extern fn zn_hip_destroy(ctx: ?*Ctx) c_int;
pub extern fn zn_hip_status_string(status: c_int) [*:0]const u8;
pub extern fn zn_hip_last_hip_error(ctx: ?*const Ctx) c_int;
pub extern fn zn_hip_device_info(ctx: ?*const Ctx, out: *DeviceInfo) c_int;
pub extern fn zn_hip_stream(ctx: ?*const Ctx) ?*anyopaque;

// ----------------------------------------------------------------- memory
pub extern fn zn_hip_alloc(ctx: ?*Ctx, bytes: usize, out: *?*anyopaque) c_int;
pub extern fn zn_hip_free(ctx: ?*Ctx, ptr: ?*anyopaque) c_int;
pub extern fn zn_hip_h2d(ctx: ?*Ctx, dst: ?*anyopaque, src: ?*const anyopaque, bytes: usize) c_int;
pub extern fn zn_hip_d2h(ctx: ?*Ctx, dst: ?*anyopaque, src: ?*const anyopaque, bytes: usize) c_int;
pub extern fn zn_hip_h2d_async(ctx: ?*Ctx, dst: ?*anyopaque, src: ?*const anyopaque, bytes: usize) c_int;
pub extern fn zn_hip_d2h_async(ctx: ?*Ctx, dst: ?*anyopaque, src: ?*const anyopaque, bytes: usize) c_int;
pub extern fn zn_hip_fill_f32(ctx: ?*Ctx, dst: ?[*]f32, value: f32, count: i64) c_int;
pub extern fn zn_hip_copy_f32(ctx: ?*Ctx, dst: ?[*]f32, src: ?[*]const f32, count: i64) c_int;
pub extern fn zn_hip_hold_stream(ctx: ?*Ctx, microseconds: f32) c_int;
pub extern fn zn_hip_sync(ctx: ?*Ctx) c_int;

// --------------------------------------------------------- graphs, events
pub extern fn zn_hip_graph_begin(ctx: ?*Ctx) c_int;
pub extern fn zn_hip_graph_end(ctx: ?*Ctx, out: *?*Graph) c_int;
pub extern fn zn_hip_graph_launch(ctx: ?*Ctx, graph: ?*Graph) c_int;
pub extern fn zn_hip_graph_destroy(graph: ?*Graph) c_int;
pub extern fn zn_hip_event_create(ctx: ?*Ctx, out: *?*Event) c_int;
pub extern fn zn_hip_event_record(ctx: ?*Ctx, ev: ?*Event) c_int;
pub extern fn zn_hip_event_elapsed_ms(start: ?*Event, end: ?*Event, ms: *f32) c_int;
pub extern fn zn_hip_event_destroy(ev: ?*Event) c_int;

// ------------------------------------------------ launch-policy overrides
pub extern fn zn_hip_set_gemm_tile(ctx: ?*Ctx, tile: c_int) c_int;
pub extern fn zn_hip_set_gemm_splits(ctx: ?*Ctx, splits: c_int) c_int;
pub extern fn zn_hip_set_gemm_persistent(ctx: ?*Ctx, mode: c_int) c_int;
pub extern fn zn_hip_set_gemm_wave_split(ctx: ?*Ctx, waves: c_int) c_int;

// ------------------------------------------------------ device pointers
pub extern fn zn_hip_sgemm(ctx: ?*Ctx, layout: c_int, m: i64, n: i64, k: i64, a: ?[*]const f32, lda: i64, b: ?[*]const f32, ldb: i64, c: ?[*]f32, ldc: i64, accumulate: c_int, bias: ?[*]const f32, act: c_int) c_int;
pub extern fn zn_hip_sgemm_noalloc(ctx: ?*Ctx, layout: c_int, m: i64, n: i64, k: i64, a: ?[*]const f32, lda: i64, b: ?[*]const f32, ldb: i64, c: ?[*]f32, ldc: i64, accumulate: c_int, bias: ?[*]const f32, act: c_int) c_int;
pub extern fn zn_hip_sgemm_strided_batched(ctx: ?*Ctx, layout: c_int, m: i64, n: i64, k: i64, a: ?[*]const f32, lda: i64, stride_a: i64, b: ?[*]const f32, ldb: i64, stride_b: i64, c: ?[*]f32, ldc: i64, stride_c: i64, batch: i64, accumulate: c_int, bias: ?[*]const f32, act: c_int) c_int;
pub extern fn zn_hip_add_bias(ctx: ?*Ctx, out: ?[*]f32, bias: ?[*]const f32, rows: i64, n: i64) c_int;
pub extern fn zn_hip_activation_forward(ctx: ?*Ctx, act: c_int, in: ?[*]const f32, out: ?[*]f32, len: i64) c_int;
pub extern fn zn_hip_activation_backward(ctx: ?*Ctx, act: c_int, y: ?[*]const f32, grad_out: ?[*]const f32, grad_in: ?[*]f32, len: i64) c_int;
pub extern fn zn_hip_accumulate_bias(ctx: ?*Ctx, grad_bias: ?[*]f32, gaa: ?[*]const f32, rows: i64, n: i64) c_int;
pub extern fn zn_hip_dense_backward(ctx: ?*Ctx, act: c_int, input: ?[*]const f32, weights: ?[*]const f32, activated_output: ?[*]const f32, grad_output: ?[*]const f32, grad_after_act: ?[*]f32, grad_input: ?[*]f32, grad_weights: ?[*]f32, grad_bias: ?[*]f32, batch: i64, in_size: i64, out_size: i64) c_int;
pub extern fn zn_hip_dense_backward_chain(ctx: ?*Ctx, act: c_int, input: ?[*]const f32, weights: ?[*]const f32, activated_output: ?[*]const f32, grad_output: ?[*]const f32, grad_after_act: ?[*]f32, grad_input: ?[*]f32, grad_weights: ?[*]f32, grad_bias: ?[*]f32, batch: i64, in_size: i64, out_size: i64, gaa_ready: c_int, prev_act: c_int, prev_activated_output: ?[*]const f32, prev_grad_after_act: ?[*]f32) c_int;
pub extern fn zn_hip_dense_pair_forward(ctx: ?*Ctx, act1: c_int, x: ?[*]const f32, w1: ?[*]const f32, b1: ?[*]const f32, h: ?[*]f32, act2: c_int, w2: ?[*]const f32, b2: ?[*]const f32, y: ?[*]f32, batch: i64, in_size: i64, hidden: i64, out_size: i64) c_int;
pub extern fn zn_hip_dense_pair_backward(ctx: ?*Ctx, act1: c_int, x: ?[*]const f32, w1: ?[*]const f32, h: ?[*]const f32, gaa1: ?[*]f32, grad_x: ?[*]f32, grad_w1: ?[*]f32, grad_b1: ?[*]f32, act2: c_int, w2: ?[*]const f32, y: ?[*]const f32, grad_y: ?[*]const f32, gaa2: ?[*]f32, grad_h: ?[*]f32, grad_w2: ?[*]f32, grad_b2: ?[*]f32, batch: i64, in_size: i64, hidden: i64, out_size: i64) c_int;
pub extern fn zn_hip_im2col(ctx: ?*Ctx, input: ?[*]const f32, col: ?[*]f32, batch: i64, channels: i64, in_h: i64, in_w: i64, k_h: i64, k_w: i64, out_h: i64, out_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64) c_int;
pub extern fn zn_hip_conv2d_forward_im2col(ctx: ?*Ctx, input: ?[*]const f32, weights: ?[*]const f32, bias: ?[*]const f32, output: ?[*]f32, batch: i64, in_channels: i64, out_channels: i64, k_h: i64, k_w: i64, in_h: i64, in_w: i64, out_h: i64, out_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64) c_int;
pub extern fn zn_hip_conv2d_forward_direct(ctx: ?*Ctx, input: ?[*]const f32, weights: ?[*]const f32, bias: ?[*]const f32, output: ?[*]f32, batch: i64, in_channels: i64, out_channels: i64, k_h: i64, k_w: i64, in_h: i64, in_w: i64, out_h: i64, out_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64) c_int;
pub extern fn zn_hip_col2im(ctx: ?*Ctx, col: ?[*]const f32, output: ?[*]f32, batch: i64, channels: i64, in_h: i64, in_w: i64, k_h: i64, k_w: i64, out_h: i64, out_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64) c_int;
pub extern fn zn_hip_conv2d_backward_im2col(ctx: ?*Ctx, input: ?[*]const f32, weights: ?[*]const f32, grad_output: ?[*]const f32, grad_input: ?[*]f32, grad_weights: ?[*]f32, grad_bias: ?[*]f32, batch: i64, in_channels: i64, out_channels: i64, k_h: i64, k_w: i64, in_h: i64, in_w: i64, out_h: i64, out_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64) c_int;
pub extern fn zn_hip_conv2d_backward_direct(ctx: ?*Ctx, input: ?[*]const f32, weights: ?[*]const f32, grad_output: ?[*]const f32, grad_input: ?[*]f32, grad_weights: ?[*]f32, grad_bias: ?[*]f32, batch: i64, in_channels: i64, out_channels: i64, k_h: i64, k_w: i64, in_h: i64, in_w: i64, out_h: i64, out_w: i64, stride_h: i64, stride_w: i64, pad_h: i64, pad_w: i64) c_int;
pub extern fn zn_hip_softmax_rows(ctx: ?*Ctx, in: ?[*]const f32, out: ?[*]f32, rows: i64, n: i64, scale: f32) c_int;
pub extern fn zn_hip_attention_forward(ctx: ?*Ctx, q: ?[*]const f32, k: ?[*]const f32, v: ?[*]const f32, out: ?[*]f32, batch: i64, seq_len: i64, d_k: i64, scale: f32) c_int;

// ------------------------------------ Backend drop-ins on host slices
pub extern fn zn_hip_mat_mul(ctx: ?*Ctx, a: ?[*]const f32, a_len: usize, b: ?[*]const f32, b_len: usize, c: ?[*]f32, c_len: usize, m: usize, n: usize, k: usize, accumulate: c_int) c_int;
pub extern fn zn_hip_mat_mul_batch(ctx: ?*Ctx, a: ?[*]const f32, a_len: usize, b: ?[*]const f32, b_len: usize, c: ?[*]f32, c_len: usize, batch_size: usize, n: usize, k: usize, accumulate: c_int) c_int;
pub extern fn zn_hip_mat_mul_transpose_a(ctx: ?*Ctx, a: ?[*]const f32, a_len: usize, b: ?[*]const f32, b_len: usize, c: ?[*]f32, c_len: usize, m: usize, n: usize, k: usize, accumulate: c_int) c_int;
pub extern fn zn_hip_mat_mul_transpose_b(ctx: ?*Ctx, a: ?[*]const f32, a_len: usize, b: ?[*]const f32, b_len: usize, c: ?[*]f32, c_len: usize, m: usize, n: usize, k: usize, accumulate: c_int) c_int;
pub extern fn zn_hip_mat_mul_bias(ctx: ?*Ctx, a: ?[*]const f32, a_len: usize, b: ?[*]const f32, b_len: usize, bias: ?[*]const f32, bias_len: usize, c: ?[*]f32, c_len: usize, batch_size: usize, n: usize, k: usize) c_int;
pub extern fn zn_hip_mat_mul_bias_relu(ctx: ?*Ctx, a: ?[*]const f32, a_len: usize, b: ?[*]const f32, b_len: usize, bias: ?[*]const f32, bias_len: usize, c: ?[*]f32, c_len: usize, batch_size: usize, n: usize, k: usize) c_int;
pub extern fn zn_hip_mat_mul_bias_sigmoid(ctx: ?*Ctx, a: ?[*]const f32, a_len: usize, b: ?[*]const f32, b_len: usize, bias: ?[*]const f32, bias_len: usize, c: ?[*]f32, c_len: usize, batch_size: usize, n: usize, k: usize) c_int;
pub extern fn zn_hip_mat_mul_bias_tanh(ctx: ?*Ctx, a: ?[*]const f32, a_len: usize, b: ?[*]const f32, b_len: usize, bias: ?[*]const f32, bias_len: usize, c: ?[*]f32, c_len: usize, batch_size: usize, n: usize, k: usize) c_int;
pub extern fn zn_hip_add_bias_host(ctx: ?*Ctx, out: ?[*]f32, out_len: usize, bias: ?[*]const f32, bias_len: usize) c_int;
pub extern fn zn_hip_activation_forward_host(ctx: ?*Ctx, act: c_int, in: ?[*]const f32, in_len: usize, out: ?[*]f32, out_len: usize) c_int;
pub extern fn zn_hip_activation_backward_host(ctx: ?*Ctx, act: c_int, y: ?[*]const f32, y_len: usize, grad_out: ?[*]const f32, grad_out_len: usize, grad_in: ?[*]f32, grad_in_len: usize) c_int;
pub extern fn zn_hip_accumulate_bias_host(ctx: ?*Ctx, grad_bias: ?[*]f32, grad_bias_len: usize, gaa: ?[*]const f32, gaa_len: usize) c_int;
pub extern fn zn_hip_conv2d_forward_host(ctx: ?*Ctx, input: ?[*]const f32, input_len: usize, weights: ?[*]const f32, weights_len: usize, bias: ?[*]const f32, bias_len: usize, output: ?[*]f32, output_len: usize, in_channels: usize, out_channels: usize, k_h: usize, k_w: usize, in_h: usize, in_w: usize, out_h: usize, out_w: usize, stride_h: usize, stride_w: usize, pad_h: usize, pad_w: usize) c_int;
pub extern fn zn_hip_conv2d_backward_host(ctx: ?*Ctx, input: ?[*]const f32, input_len: usize, weights: ?[*]const f32, weights_len: usize, grad_output: ?[*]const f32, grad_output_len: usize, grad_input: ?[*]f32, grad_input_len: usize, grad_weights: ?[*]f32, grad_weights_len: usize, grad_bias: ?[*]f32, grad_bias_len: usize, in_channels: usize, out_channels: usize, k_h: usize, k_w: usize, in_h: usize, in_w: usize, out_h: usize, out_w: usize, stride_h: usize, stride_w: usize, pad_h: usize, pad_w: usize) c_int;
pub extern fn zn_hip_attention_forward_host(ctx: ?*Ctx, q: ?[*]const f32, q_len: usize, k: ?[*]const f32, k_len: usize, v: ?[*]const f32, v_len: usize, output: ?[*]f32, output_len: usize, scores: ?[*]f32, scores_len: usize, seq_len: usize, d_k: usize, scale: f32) c_int;

// ------------------------------------------------------------- Zig side

pub const HipError = error{ NoDevice, CodeObject, Symbol, InvalidArgument, OutOfMemory, Launch, Hip, Overflow, Unknown };

/// Status -> Zig error, the role of checkCuda (src/cuda_driver.zig:1119-1160).
pub fn check(status: c_int) HipError!void {
    return switch (status) {
        0 => {},
        -1 => error.NoDevice,
        -2 => error.CodeObject,
        -3 => error.Symbol,
        -4 => error.InvalidArgument,
        -5 => error.OutOfMemory,
        -6 => error.Launch,
        -7 => error.Hip,
        -8 => error.Overflow,
        else => error.Unknown,
    };
}

/// The epilogue id of an activation the GPU path applies (linear, relu,
/// sigmoid, tanh); the others (softmax, gelu, leaky_relu, elu) stay on the
/// CPU arm.
pub fn actId(act: activation.Activation) ?c_int {
    return switch (act) {
        .linear => @intFromEnum(Act.linear),
        .relu => @intFromEnum(Act.relu),
        .sigmoid => @intFromEnum(Act.sigmoid),
        .tanh => @intFromEnum(Act.tanh),
        else => null,
    };
}

/// The GEMM-family operators of `Backend` on one MI355X: each method takes
/// the reference method's slices and scalars (without the Metal buffers) and
/// returns when the outputs are in host memory, like CudaBackend's
/// synchronous arms (src/cuda.zig:617).  One instance serves one thread.
pub const HipBackend = struct {
    ctx: *Ctx,

    /// CudaBackend.isAvailable (src/cuda.zig:317-328).
    pub fn isAvailable() bool {
        return zn_hip_available() == 1;
    }

    /// The context on `device`; code objects from $ZN_HIP_CODE_OBJECT_DIR or
    /// the directory of libzn_hip.
    pub fn init(device: c_int) HipError!HipBackend {
        var ctx: ?*Ctx = null;
        try check(zn_hip_create(device, null, &ctx));
        return .{ .ctx = ctx.? };
    }

    pub fn deinit(self: *HipBackend) void {
        _ = zn_hip_destroy(self.ctx);
    }

    pub fn matMul(self: *HipBackend, a: []const f32, b: []const f32, c: []f32, m: usize, n: usize, k: usize, accumulate: bool) HipError!void {
        try check(zn_hip_mat_mul(self.ctx, a.ptr, a.len, b.ptr, b.len, c.ptr, c.len, m, n, k, @intFromBool(accumulate)));
    }
    pub fn matMulBatch(self: *HipBackend, a: []const f32, b: []const f32, c: []f32, batch_size: usize, n: usize, k: usize, accumulate: bool) HipError!void {
        try check(zn_hip_mat_mul_batch(self.ctx, a.ptr, a.len, b.ptr, b.len, c.ptr, c.len, batch_size, n, k, @intFromBool(accumulate)));
    }
    pub fn matMulTransposeA(self: *HipBackend, a: []const f32, b: []const f32, c: []f32, m: usize, n: usize, k: usize, accumulate: bool) HipError!void {
        try check(zn_hip_mat_mul_transpose_a(self.ctx, a.ptr, a.len, b.ptr, b.len, c.ptr, c.len, m, n, k, @intFromBool(accumulate)));
    }
    pub fn matMulTransposeB(self: *HipBackend, a: []const f32, b: []const f32, c: []f32, m: usize, n: usize, k: usize, accumulate: bool) HipError!void {
        try check(zn_hip_mat_mul_transpose_b(self.ctx, a.ptr, a.len, b.ptr, b.len, c.ptr, c.len, m, n, k, @intFromBool(accumulate)));
    }
    pub fn matMulBias(self: *HipBackend, a: []const f32, b: []const f32, bias: []const f32, c: []f32, batch_size: usize, n: usize, k: usize) HipError!void {
        try check(zn_hip_mat_mul_bias(self.ctx, a.ptr, a.len, b.ptr, b.len, bias.ptr, bias.len, c.ptr, c.len, batch_size, n, k));
    }
    pub fn matMulBiasRelu(self: *HipBackend, a: []const f32, b: []const f32, bias: []const f32, c: []f32, batch_size: usize, n: usize, k: usize) HipError!void {
        try check(zn_hip_mat_mul_bias_relu(self.ctx, a.ptr, a.len, b.ptr, b.len, bias.ptr, bias.len, c.ptr, c.len, batch_size, n, k));
    }
    pub fn matMulBiasSigmoid(self: *HipBackend, a: []const f32, b: []const f32, bias: []const f32, c: []f32, batch_size: usize, n: usize, k: usize) HipError!void {
        try check(zn_hip_mat_mul_bias_sigmoid(self.ctx, a.ptr, a.len, b.ptr, b.len, bias.ptr, bias.len, c.ptr, c.len, batch_size, n, k));
    }
    pub fn matMulBiasTanh(self: *HipBackend, a: []const f32, b: []const f32, bias: []const f32, c: []f32, batch_size: usize, n: usize, k: usize) HipError!void {
        try check(zn_hip_mat_mul_bias_tanh(self.ctx, a.ptr, a.len, b.ptr, b.len, bias.ptr, bias.len, c.ptr, c.len, batch_size, n, k));
    }
    pub fn addBias(self: *HipBackend, output: []f32, bias: []const f32) HipError!void {
        try check(zn_hip_add_bias_host(self.ctx, output.ptr, output.len, bias.ptr, bias.len));
    }
    pub fn accumulateBias(self: *HipBackend, grad_bias: []f32, grad_after_act: []const f32) HipError!void {
        try check(zn_hip_accumulate_bias_host(self.ctx, grad_bias.ptr, grad_bias.len, grad_after_act.ptr, grad_after_act.len));
    }
    /// `act` from actId (linear, relu, sigmoid, tanh).
    pub fn activationForward(self: *HipBackend, act: c_int, input: []const f32, output: []f32) HipError!void {
        try check(zn_hip_activation_forward_host(self.ctx, act, input.ptr, input.len, output.ptr, output.len));
    }
    /// `input` is the activated output y, as in Backend.activationBackward.
    pub fn activationBackward(self: *HipBackend, act: c_int, input: []const f32, grad_output: []const f32, grad_input: []f32) HipError!void {
        try check(zn_hip_activation_backward_host(self.ctx, act, input.ptr, input.len, grad_output.ptr, grad_output.len, grad_input.ptr, grad_input.len));
    }
    /// Keeps the reference's im2col-or-direct switch (src/backend.zig:3009-3016).
    pub fn conv2dForward(self: *HipBackend, input: []const f32, weights: []const f32, bias: []const f32, output: []f32, in_channels: usize, out_channels: usize, kernel_h: usize, kernel_w: usize, input_h: usize, input_w: usize, output_h: usize, output_w: usize, stride_h: usize, stride_w: usize, padding_h: usize, padding_w: usize) HipError!void {
        try check(zn_hip_conv2d_forward_host(self.ctx, input.ptr, input.len, weights.ptr, weights.len, bias.ptr, bias.len, output.ptr, output.len, in_channels, out_channels, kernel_h, kernel_w, input_h, input_w, output_h, output_w, stride_h, stride_w, padding_h, padding_w));
    }
    /// Keeps the reference's im2col-or-direct switch (src/backend.zig:3053-3062).
    pub fn conv2dBackward(self: *HipBackend, input: []const f32, weights: []const f32, grad_output: []const f32, grad_input: []f32, grad_weights: []f32, grad_bias: []f32, in_channels: usize, out_channels: usize, kernel_h: usize, kernel_w: usize, input_h: usize, input_w: usize, output_h: usize, output_w: usize, stride_h: usize, stride_w: usize, padding_h: usize, padding_w: usize) HipError!void {
        try check(zn_hip_conv2d_backward_host(self.ctx, input.ptr, input.len, weights.ptr, weights.len, grad_output.ptr, grad_output.len, grad_input.ptr, grad_input.len, grad_weights.ptr, grad_weights.len, grad_bias.ptr, grad_bias.len, in_channels, out_channels, kernel_h, kernel_w, input_h, input_w, output_h, output_w, stride_h, stride_w, padding_h, padding_w));
    }
    pub fn attentionForward(self: *HipBackend, q: []const f32, k: []const f32, v: []const f32, output: []f32, scores_buffer: []f32, seq_len: usize, d_k: usize, scaling_factor: f32) HipError!void {
        try check(zn_hip_attention_forward_host(self.ctx, q.ptr, q.len, k.ptr, k.len, v.ptr, v.len, output.ptr, output.len, scores_buffer.ptr, scores_buffer.len, seq_len, d_k, scaling_factor));
    }

    // --- device-resident tensors (asynchronous on the context's stream)

    pub fn alloc(self: *HipBackend, count: usize) HipError![*]f32 {
        var p: ?*anyopaque = null;
        try check(zn_hip_alloc(self.ctx, count * @sizeOf(f32), &p));
        return @ptrCast(@alignCast(p.?));
    }
    pub fn free(self: *HipBackend, ptr: [*]f32) void {
        _ = zn_hip_free(self.ctx, ptr);
    }
    pub fn upload(self: *HipBackend, dst: [*]f32, src: []const f32) HipError!void {
        try check(zn_hip_h2d(self.ctx, dst, src.ptr, src.len * @sizeOf(f32)));
    }
    pub fn download(self: *HipBackend, dst: []f32, src: [*]const f32) HipError!void {
        try check(zn_hip_d2h(self.ctx, dst.ptr, src, dst.len * @sizeOf(f32)));
    }
    pub fn sync(self: *HipBackend) HipError!void {
        try check(zn_hip_sync(self.ctx));
    }
    /// C = act((accumulate ? C : 0) + op(A).op(B) + bias), explicit leading dimensions.
    pub fn sgemm(self: *HipBackend, layout: Layout, m: i64, n: i64, k: i64, a: [*]const f32, lda: i64, b: [*]const f32, ldb: i64, c: [*]f32, ldc: i64, accumulate: bool, bias: ?[*]const f32, act: Act) HipError!void {
        try check(zn_hip_sgemm(self.ctx, @intFromEnum(layout), m, n, k, a, lda, b, ldb, c, ldc, @intFromBool(accumulate), bias, @intFromEnum(act)));
    }
    /// sgemm for callers that cannot allocate (e.g. while a graph is captured).
    pub fn sgemmNoAlloc(self: *HipBackend, layout: Layout, m: i64, n: i64, k: i64, a: [*]const f32, lda: i64, b: [*]const f32, ldb: i64, c: [*]f32, ldc: i64, accumulate: bool, bias: ?[*]const f32, act: Act) HipError!void {
        try check(zn_hip_sgemm_noalloc(self.ctx, @intFromEnum(layout), m, n, k, a, lda, b, ldb, c, ldc, @intFromBool(accumulate), bias, @intFromEnum(act)));
    }
    pub fn sgemmStridedBatched(self: *HipBackend, layout: Layout, m: i64, n: i64, k: i64, a: [*]const f32, lda: i64, stride_a: i64, b: [*]const f32, ldb: i64, stride_b: i64, c: [*]f32, ldc: i64, stride_c: i64, batch: i64, accumulate: bool, bias: ?[*]const f32, act: Act) HipError!void {
        try check(zn_hip_sgemm_strided_batched(self.ctx, @intFromEnum(layout), m, n, k, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c, batch, @intFromBool(accumulate), bias, @intFromEnum(act)));
    }
    /// Dense.backward (src/layer.zig:411-475) on device pointers; grad_input
    /// null for a first layer.
    pub fn denseBackward(self: *HipBackend, act: Act, input: [*]const f32, weights: [*]const f32, activated_output: [*]const f32, grad_output: [*]const f32, grad_after_act: [*]f32, grad_input: ?[*]f32, grad_weights: [*]f32, grad_bias: [*]f32, batch: i64, in_size: i64, out_size: i64) HipError!void {
        try check(zn_hip_dense_backward(self.ctx, @intFromEnum(act), input, weights, activated_output, grad_output, grad_after_act, grad_input, grad_weights, grad_bias, batch, in_size, out_size));
    }
    /// denseBackward for layers walked top-down: with gaa_ready the layer's
    /// grad_after_act was written by the call of the layer above (y and
    /// grad_output unread); a non-null prev_grad_after_act also receives the
    /// layer below's activation derivative.  Same bits as denseBackward.
    pub fn denseBackwardChain(self: *HipBackend, act: Act, input: [*]const f32, weights: [*]const f32, activated_output: ?[*]const f32, grad_output: ?[*]const f32, grad_after_act: [*]f32, grad_input: ?[*]f32, grad_weights: [*]f32, grad_bias: [*]f32, batch: i64, in_size: i64, out_size: i64, gaa_ready: bool, prev_act: Act, prev_activated_output: ?[*]const f32, prev_grad_after_act: ?[*]f32) HipError!void {
        try check(zn_hip_dense_backward_chain(self.ctx, @intFromEnum(act), input, weights, activated_output, grad_output, grad_after_act, grad_input, grad_weights, grad_bias, batch, in_size, out_size, @intFromBool(gaa_ready), @intFromEnum(prev_act), prev_activated_output, prev_grad_after_act));
    }
    /// Two stacked Dense forwards (Network.forward over a lower layer and a
    /// narrow top layer): one launch when the top layer has at most 16 outputs.
    pub fn densePairForward(self: *HipBackend, act1: Act, x: [*]const f32, w1: [*]const f32, b1: ?[*]const f32, h: [*]f32, act2: Act, w2: [*]const f32, b2: ?[*]const f32, y: [*]f32, batch: i64, in_size: i64, hidden: i64, out_size: i64) HipError!void {
        try check(zn_hip_dense_pair_forward(self.ctx, @intFromEnum(act1), x, w1, b1, h, @intFromEnum(act2), w2, b2, y, batch, in_size, hidden, out_size));
    }
    /// The backward of the same pair, top layer first, in one launch under
    /// the same limit; grad_x may be null (the network's first layer).
    pub fn densePairBackward(self: *HipBackend, act1: Act, x: [*]const f32, w1: [*]const f32, h: [*]const f32, gaa1: [*]f32, grad_x: ?[*]f32, grad_w1: [*]f32, grad_b1: [*]f32, act2: Act, w2: [*]const f32, y: [*]const f32, grad_y: [*]const f32, gaa2: [*]f32, grad_h: [*]f32, grad_w2: [*]f32, grad_b2: [*]f32, batch: i64, in_size: i64, hidden: i64, out_size: i64) HipError!void {
        try check(zn_hip_dense_pair_backward(self.ctx, @intFromEnum(act1), x, w1, h, gaa1, grad_x, grad_w1, grad_b1, @intFromEnum(act2), w2, y, grad_y, gaa2, grad_h, grad_w2, grad_b2, batch, in_size, hidden, out_size));
    }
    pub fn attentionForwardDevice(self: *HipBackend, q: [*]const f32, k: [*]const f32, v: [*]const f32, out: [*]f32, batch: i64, seq_len: i64, d_k: i64, scale: f32) HipError!void {
        try check(zn_hip_attention_forward(self.ctx, q, k, v, out, batch, seq_len, d_k, scale));
    }

    // --- HIP graphs of device-pointer calls (run the sequence once first)

    pub fn graphBegin(self: *HipBackend) HipError!void {
        try check(zn_hip_graph_begin(self.ctx));
    }
    pub fn graphEnd(self: *HipBackend) HipError!*Graph {
        var g: ?*Graph = null;
        try check(zn_hip_graph_end(self.ctx, &g));
        return g.?;
    }
    pub fn graphLaunch(self: *HipBackend, graph: *Graph) HipError!void {
        try check(zn_hip_graph_launch(self.ctx, graph));
    }
    pub fn graphDestroy(graph: *Graph) void {
        _ = zn_hip_graph_destroy(graph);
    }
};
