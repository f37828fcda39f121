//! gpu_hip.zig -- the MI355X (gfx950) backend of the Zig Gemma engine, behind
//! the call surface of the Vulkan module it replaces.
//!
//! Install it as src/gpu.zig of Sullux/ai-research, in place of the Vulkan
//! module (src/gpu.zig with src/gpu/ and shaders/), and link the backend
//! library (build.zig wiring in INTEGRATION.md).  Every name the engine's
//! call sites use keeps its path and signature, so these files stay as they
//! are:
//!   src/main.zig:83-101        gpu.context.GpuContext.init / .deinit / .device_name,
//!                              gpu.model_gpu.GpuModelContext.init / .deinit
//!   src/model/forward.zig:41-45 gpu.model_dispatch.gpuDispatchForwardToken
//!   src/model/bench.zig:12-15   g.engine.submitPreRecorded(g.cmd_buf_decode)
//!   src/interactive.zig, src/server.zig, src/model/loader.zig: the
//!                              gpu.model_gpu.GpuModelContext type
//! The C ABI is include/gemma_hip.h; each function used here names the
//! reference interface it replaces.  tests/c_host/decode_host.c runs this
//! file's call sequence in C, including the --bench replays.
//!
//! Not built in this repository: the image has no Zig toolchain.  Written for
//! Zig 0.14 (README.md:87 of the reference).
const std = @import("std");
const c = @cImport(@cInclude("gemma_hip.h"));
const model_types = @import("model/types.zig");
const loader = @import("model/loader.zig");
pub const quant = @import("quant.zig");

/// The backend's status codes as Zig errors (in place of the Vulkan set:
/// VulkanLibraryNotFound, NoVulkanDevices, Vk*Failed; src/gpu/vk_api.zig:113,
/// src/gpu/context.zig:24-68, src/gpu/buffer.zig:20-44).
pub const Error = error{ NoDevice, CodeObject, Alloc, Invalid, Unsupported, Hip };

fn check(st: c.gh_status) Error!void {
    return switch (st) {
        c.GH_OK => {},
        c.GH_ERR_NO_DEVICE => error.NoDevice,
        c.GH_ERR_CODE_OBJECT => error.CodeObject,
        c.GH_ERR_ALLOC => error.Alloc,
        c.GH_ERR_INVALID => error.Invalid,
        c.GH_ERR_UNSUPPORTED => error.Unsupported,
        else => error.Hip,
    };
}

fn bf16Ptr(s: anytype) [*c]const u16 {
    return @ptrCast(s.ptr);
}

fn optBf16Ptr(s: anytype) [*c]const u16 {
    return switch (@typeInfo(@TypeOf(s))) {
        .optional => if (s) |v| (if (v.len == 0) null else bf16Ptr(v)) else null,
        else => if (s.len == 0) null else bf16Ptr(s),
    };
}

/// src/gpu/context.zig:13-104
pub const context = struct {
    pub const GpuContext = struct {
        h: *c.gh_context,
        device_name: [256]u8,

        /// GpuContext.init (context.zig:17): device 0, gfx950 code objects
        /// from the directory holding libgemma_hip.so.
        pub fn init(allocator: std.mem.Allocator) Error!GpuContext {
            _ = allocator;
            var h: ?*c.gh_context = null;
            try check(c.gh_context_init(null, &h));
            var self = GpuContext{ .h = h.?, .device_name = [_]u8{0} ** 256 };
            const name = std.mem.span(c.gh_context_device_name(self.h));
            const n = @min(name.len, self.device_name.len - 1);
            @memcpy(self.device_name[0..n], name[0..n]);
            return self;
        }

        /// GpuContext.deinit (context.zig:104).
        pub fn deinit(self: *GpuContext) void {
            c.gh_context_deinit(self.h);
        }
    };
};

/// src/gpu/model_gpu.zig:35-197
pub const model_gpu = struct {
    /// A pre-recorded command buffer: one of the model's two recorded graphs
    /// (cmd_buf_decode and cmd_buf_prefill, model_gpu.zig:182-183).
    pub const CommandBuffer = c.gh_graph_kind;

    /// The part of GpuEngine (src/gpu/kernels.zig:14-157) the engine's callers
    /// use outside the backend: submitPreRecorded (kernels.zig:147-157),
    /// which --bench calls with cmd_buf_decode (src/model/bench.zig:12-15).
    pub const Engine = struct {
        model: *c.gh_model,

        /// Replays the graph on the inputs the device holds (those of the
        /// last forward call) and waits for it, as the reference submits the
        /// command buffer and waits on its fence.
        pub fn submitPreRecorded(self: *const Engine, cmd_buf: CommandBuffer) Error!void {
            try check(c.gh_model_submit_prerecorded(self.model, cmd_buf));
        }
    };

    pub const GpuModelContext = struct {
        h: *c.gh_model,
        engine: Engine,
        cmd_buf_decode: CommandBuffer,
        cmd_buf_prefill: CommandBuffer,

        /// GpuModelContext.init (model_gpu.zig:75): quantizes the borrowed
        /// bf16 weights with quant.zig's bytes (or keeps them in mode .none),
        /// allocates the per-layer K/V caches and records the decode graph
        /// gated at quiescence_thresh and the prefill graph at 0.
        pub fn init(allocator: std.mem.Allocator, ctx: *const context.GpuContext, m: *const loader.Model,
                    config: model_types.ModelConfig, mode: quant.QuantMode, quiescence_thresh: f32) Error!GpuModelContext {
            _ = allocator;
            if (config.num_hidden_layers > 64) return error.Unsupported;
            var cfg = std.mem.zeroes(c.gh_model_config);
            cfg.vocab_size = @intCast(config.vocab_size);
            cfg.hidden_size = @intCast(config.hidden_size);
            cfg.intermediate_size = @intCast(config.intermediate_size);
            cfg.num_hidden_layers = @intCast(config.num_hidden_layers);
            cfg.num_attention_heads = @intCast(config.num_attention_heads);
            cfg.num_key_value_heads = @intCast(config.num_key_value_heads);
            cfg.num_global_key_value_heads = @intCast(config.num_global_key_value_heads);
            cfg.head_dim = @intCast(config.head_dim);
            cfg.global_head_dim = @intCast(config.global_head_dim);
            cfg.attention_k_eq_v = @intFromBool(config.attention_k_eq_v);
            // the reference's per-layer cache depth (model_gpu.zig:86); the
            // ring (anchors + window + recall, src/main.zig:34) lives in its
            // first slots, and the attention runs splits by the active count
            cfg.max_slots = 1024;
            cfg.rms_norm_eps = config.rms_norm_eps;
            cfg.rope_theta = config.rope_theta;
            cfg.rope_theta_full = config.rope_theta_full;
            for (0..config.num_hidden_layers) |i|
                cfg.layer_types[i] = @intFromBool(config.layer_types[i] == .full_attention);

            // borrowed bf16 pointers, valid for the duration of the call
            var lw: [64]c.gh_layer_weights = undefined;
            for (m.layers, 0..) |l, i| lw[i] = .{
                .input_layernorm = bf16Ptr(l.input_layernorm),
                .q_proj = bf16Ptr(l.q_proj),
                .k_proj = bf16Ptr(l.k_proj),
                .v_proj = optBf16Ptr(l.v_proj), // absent: the key projection serves as value (model_gpu.zig:124)
                .o_proj = bf16Ptr(l.o_proj),
                .q_norm = bf16Ptr(l.q_norm),
                .k_norm = optBf16Ptr(l.k_norm), // absent: ones (model_gpu.zig:64-73)
                .post_attention_layernorm = optBf16Ptr(l.post_attention_layernorm),
                .pre_feedforward_layernorm = bf16Ptr(l.pre_feedforward_layernorm),
                .gate_proj = bf16Ptr(l.gate_proj),
                .up_proj = bf16Ptr(l.up_proj),
                .down_proj = bf16Ptr(l.down_proj),
                .post_feedforward_layernorm = optBf16Ptr(l.post_feedforward_layernorm),
                .layer_scalar = l.layer_scalar orelse 1.0,
            };
            const qm: c.gh_quant_mode = switch (mode) {
                .q4 => @intCast(c.GH_QUANT_Q4),
                .q8 => @intCast(c.GH_QUANT_Q8),
                .none => @intCast(c.GH_QUANT_NONE),
            };
            var h: ?*c.gh_model = null;
            try check(c.gh_model_init(ctx.h, &cfg, &lw, bf16Ptr(m.embed_tokens), bf16Ptr(m.final_norm),
                                      qm, quiescence_thresh, &h));
            return .{
                .h = h.?,
                .engine = .{ .model = h.? },
                .cmd_buf_decode = @intCast(c.GH_GRAPH_DECODE),
                .cmd_buf_prefill = @intCast(c.GH_GRAPH_PREFILL),
            };
        }

        /// GpuModelContext.deinit (model_gpu.zig:187).
        pub fn deinit(self: *GpuModelContext) void {
            c.gh_model_deinit(self.h);
        }
    };
};

/// src/gpu/model_dispatch.zig:131-147
pub const model_dispatch = struct {
    /// gpuDispatchForwardToken: same arguments, same result.  logits.len >= V
    /// selects the decode graph (LM head + argmax) and returns the greedy
    /// token; otherwise the prefill graph runs and 0 comes back.  Logits stay
    /// on the device, as in the reference.
    pub fn gpuDispatchForwardToken(gpu: *model_gpu.GpuModelContext, config: *const model_types.ModelConfig,
                                   layers: []const model_types.LayerWeights, x: []const f32, logits: []f32,
                                   clock: usize, slot_idx: usize, active_slots: []const usize) u32 {
        _ = layers;
        var act: [1024]u32 = undefined;
        if (active_slots.len > act.len) {
            std.log.err("gpuDispatchForwardToken: {d} active slots exceed the 1024-slot cache", .{active_slots.len});
            return 0;
        }
        for (act[0..active_slots.len], active_slots) |*d, s| d.* = @intCast(s);
        var token: u32 = 0;
        const want_logits: c_int = @intFromBool(logits.len >= config.vocab_size);
        check(c.gh_dispatch_forward_token(gpu.h, x.ptr, want_logits, clock, @intCast(slot_idx), &act,
                                          @intCast(active_slots.len), &token)) catch |err| {
            std.log.err("gh_dispatch_forward_token: {} ({s})", .{ err, c.gh_last_error() });
            return 0; // the reference's result on a failed submit (model_dispatch.zig:145)
        };
        return token;
    }
};

test "hip context initialization" {
    var ctx = context.GpuContext.init(std.testing.allocator) catch |err| {
        if (err == error.NoDevice) return;
        return err;
    };
    defer ctx.deinit();
    try std.testing.expect(ctx.device_name[0] != 0);
}
