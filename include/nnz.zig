//! nnz.zig -- Zig binding of include/nnz.h for nnmetal's host code.
//!
//! What a maintainer of nnmetal (duanebester/nnzap) adds to call the MI355X
//! library instead of the Metal shaders: the `dispatch*` helpers of
//! nnmetal/src/transformer.zig:384-2387 keep their names and argument roles,
//! with two mechanical changes at every call site --
//!
//!   * `device: *const metal.Device, encoder: objc.Object` becomes one
//!     `ctx: Ctx` (an nnz_ctx owning a HIP stream; launches run in call
//!     order, so the reference's explicit barriers, transformer.zig:2830-2888,
//!     disappear);
//!   * MTLBuffers become device pointers (`Buf(T)`), PackedBuffer / Q4Buffer
//!     (metal.zig:227-469) become `QWeight`.
//!
//! The dims structs are the reference's own extern structs, imported from the
//! C header (field for field, transformer.zig:389-479).  Preconditions the
//! reference asserts come back as `error.Nnz*` with nnz_last_error().
//!
//! build.zig (the reference links Metal/Foundation/CoreGraphics at
//! nnmetal/build.zig:20-23; these lines replace them):
//!
//!     const nnz = b.addModule("nnz", .{ .root_source_file = b.path("nnz.zig") });
//!     nnz.addIncludePath(b.path("include"));
//!     nnz.addLibraryPath(b.path("nnzap_amd"));
//!     nnz.linkSystemLibrary("nnzap_amd", .{});
//!     exe.root_module.addImport("nnz", nnz);
//!
//! No Zig toolchain exists in this build's image, so this file is not
//! compiled here; tests/c/abi_check.c compiles the same header from C and
//! pins the struct layouts this binding relies on.
const std = @import("std");

pub const c = @cImport(@cInclude("nnz.h"));

pub const Error = error{
    NnzInvalid,
    NnzUnsupported,
    NnzHip,
    NnzOutOfMemory,
    NnzTimeout,
    NnzState,
};

fn err_of(rc: c_int) Error {
    return switch (rc) {
        c.NNZ_EINVAL => error.NnzInvalid,
        c.NNZ_EUNSUPPORTED => error.NnzUnsupported,
        c.NNZ_ENOMEM => error.NnzOutOfMemory,
        c.NNZ_ETIMEOUT => error.NnzTimeout,
        c.NNZ_ESTATE => error.NnzState,
        else => error.NnzHip,
    };
}

// Dims structs: the reference's extern structs (transformer.zig:389-479).
pub const RMSNormDims = c.nnz_rmsnorm_dims;
pub const RoPEDims = c.nnz_rope_dims;
pub const KVUpdateDims = c.nnz_kv_update_dims;
pub const FusedRoPEKVDims = c.nnz_fused_rope_kv_dims;
pub const FusedNormRoPEDims = c.nnz_fused_norm_rope_dims;
pub const FusedKNormRoPEKVDims = c.nnz_fused_k_norm_rope_kv_dims;
pub const GQADims = c.nnz_gqa_dims;
pub const GQAFusedDims = c.nnz_gqa_fused_dims;
pub const EmbedDims = c.nnz_embed_dims;
pub const QMVDims = c.nnz_qmv_dims;

/// Replaces metal.Device (metal.zig:839-1372): device + command queue.
pub const Ctx = struct {
    raw: *c.nnz_ctx,

    /// Device.init (metal.zig:959-1020).  `stream` null: the library creates
    /// its own non-blocking stream.
    pub fn init(device: c_int, stream: ?*anyopaque) Error!Ctx {
        var raw: ?*c.nnz_ctx = null;
        const rc = c.nnz_ctx_create(device, stream, &raw);
        if (rc != c.NNZ_OK) return err_of(rc);
        return .{ .raw = raw.? };
    }

    pub fn deinit(self: Ctx) void {
        _ = c.nnz_ctx_destroy(self.raw);
    }

    pub fn check(self: Ctx, rc: c_int) Error!void {
        if (rc == c.NNZ_OK) return;
        std.log.err("nnz: {s}", .{c.nnz_last_error(self.raw)});
        return err_of(rc);
    }

    /// commitAndWait / commitAndSpinOnFlag (metal.zig:1293-1352), bounded.
    pub fn sync(self: Ctx, timeout_ms: u32) Error!void {
        try self.check(c.nnz_stream_sync(self.raw, timeout_ms));
    }

    /// Buffer.init (metal.zig:80-140): zero-filled device memory.
    pub fn alloc(self: Ctx, comptime T: type, n: usize) Error!Buf(T) {
        var p: ?*anyopaque = null;
        try self.check(c.nnz_alloc(self.raw, n * @sizeOf(T), &p));
        return .{ .ptr = @ptrCast(@alignCast(p.?)), .len = n };
    }

    pub fn free(self: Ctx, buf: anytype) void {
        _ = c.nnz_free(self.raw, @ptrCast(buf.ptr));
    }

    /// The one-time copy that replaces writes into shared memory.
    pub fn upload(self: Ctx, comptime T: type, dst: Buf(T), src: []const T) Error!void {
        std.debug.assert(src.len <= dst.len);
        try self.check(c.nnz_upload(self.raw, @ptrCast(dst.ptr), @ptrCast(src.ptr), src.len * @sizeOf(T)));
    }

    pub fn download(self: Ctx, comptime T: type, dst: []T, src: Buf(T)) Error!void {
        std.debug.assert(dst.len <= src.len);
        try self.check(c.nnz_download(self.raw, @ptrCast(dst.ptr), @ptrCast(src.ptr), dst.len * @sizeOf(T)));
    }
};

/// A typed device pointer (the role of metal.Buffer / HalfBuffer).
pub fn Buf(comptime T: type) type {
    return struct {
        ptr: [*]T,
        len: usize,

        pub fn raw(self: @This()) ?*anyopaque {
            return @ptrCast(self.ptr);
        }
    };
}

/// PackedBuffer (metal.zig:227-335, bits 1) / Q4Buffer (:337-469, bits 4).
pub const QWeight = c.nnz_qweight;

pub fn packedWeight(codes: ?*const anyopaque, scales: ?*const anyopaque, m: u32, k: u32, group_size: u32) QWeight {
    return .{ .codes = codes, .scales = scales, .biases = null, .packed_count = m * k, .group_size = group_size, .bits = 1, .scale_dtype = c.NNZ_F16 };
}

pub fn q4Weight(codes: ?*const anyopaque, scales: ?*const anyopaque, biases: ?*const anyopaque, m: u32, k: u32, group_size: u32) QWeight {
    return .{ .codes = codes, .scales = scales, .biases = biases, .packed_count = m * k, .group_size = group_size, .bits = 4, .scale_dtype = c.NNZ_BF16 };
}

// ---- QMV family (transformer.zig:1120-1893) --------------------------------

/// transformer.zig:1565 dispatchQMV
pub fn dispatchQMV(ctx: Ctx, w: *const QWeight, input: Buf(f32), output: Buf(f32), dims: QMVDims) Error!void {
    try ctx.check(c.nnz_dispatch_qmv(ctx.raw, w, input.ptr, output.ptr, dims));
}

/// transformer.zig:1653 dispatchQMVf16in (LM head: half in, f32 out)
pub fn dispatchQMVf16in(ctx: Ctx, w: *const QWeight, input: Buf(f16), output: Buf(f32), dims: QMVDims) Error!void {
    try ctx.check(c.nnz_dispatch_qmv_f16in(ctx.raw, w, input.raw(), output.ptr, dims));
}

/// transformer.zig:1728 dispatchQMVf16io
pub fn dispatchQMVf16io(ctx: Ctx, w: *const QWeight, input: Buf(f16), output: Buf(f16), dims: QMVDims) Error!void {
    try ctx.check(c.nnz_dispatch_qmv_f16io(ctx.raw, w, input.raw(), output.raw(), dims));
}

/// transformer.zig:1806 dispatchQMVf16ioResadd (residual[r] += W x)
pub fn dispatchQMVf16ioResadd(ctx: Ctx, w: *const QWeight, input: Buf(f16), residual: Buf(f32), dims: QMVDims) Error!void {
    try ctx.check(c.nnz_dispatch_qmv_f16io_resadd(ctx.raw, w, input.raw(), residual.ptr, dims));
}

/// transformer.zig:1238 dispatchQMVFusedPairf16io
pub fn dispatchQMVFusedPairf16io(ctx: Ctx, wa: *const QWeight, wb: *const QWeight, input: Buf(f16), out_a: Buf(f16), out_b: Buf(f16), dims: QMVDims) Error!void {
    try ctx.check(c.nnz_dispatch_qmv_fused_pair_f16io(ctx.raw, wa, wb, input.raw(), out_a.raw(), out_b.raw(), dims));
}

/// transformer.zig:1309 dispatchQMVFusedPairSiLUf16io (silu(Wg x) * (Wu x))
pub fn dispatchQMVFusedPairSiLUf16io(ctx: Ctx, w_gate: *const QWeight, w_up: *const QWeight, input: Buf(f16), output: Buf(f16), dims: QMVDims) Error!void {
    try ctx.check(c.nnz_dispatch_qmv_fused_pair_silu_f16io(ctx.raw, w_gate, w_up, input.raw(), output.raw(), dims));
}

/// transformer.zig:1373 dispatchFusedNormPairSiLUf16io (RMSNorm fused in)
pub fn dispatchFusedNormPairSiLUf16io(ctx: Ctx, w_gate: *const QWeight, w_up: *const QWeight, residual: Buf(f32), output: Buf(f16), norm_scale: Buf(f32), dims: QMVDims) Error!void {
    try ctx.check(c.nnz_dispatch_fused_norm_pair_silu_f16io(ctx.raw, w_gate, w_up, residual.ptr, output.raw(), norm_scale.ptr, dims));
}

/// transformer.zig:1438 dispatchFusedNormQMVf16io
pub fn dispatchFusedNormQMVf16io(ctx: Ctx, w: *const QWeight, residual: Buf(f32), output: Buf(f16), norm_scale: Buf(f32), dims: QMVDims) Error!void {
    try ctx.check(c.nnz_dispatch_fused_norm_qmv_f16io(ctx.raw, w, residual.ptr, output.raw(), norm_scale.ptr, dims));
}

/// transformer.zig:1501 dispatchFusedNormPairQMVf16io
pub fn dispatchFusedNormPairQMVf16io(ctx: Ctx, wa: *const QWeight, wb: *const QWeight, residual: Buf(f32), out_a: Buf(f16), out_b: Buf(f16), norm_scale: Buf(f32), dims: QMVDims) Error!void {
    try ctx.check(c.nnz_dispatch_fused_norm_pair_qmv_f16io(ctx.raw, wa, wb, residual.ptr, out_a.raw(), out_b.raw(), norm_scale.ptr, dims));
}

/// encodeAttnProjFusedNorm (transformer.zig:3024-3083) as one launch
pub fn dispatchFusedNormQKVf16io(ctx: Ctx, wq: *const QWeight, wk: *const QWeight, wv: *const QWeight, residual: Buf(f32), q: Buf(f16), k: Buf(f16), v: Buf(f16), norm_scale: Buf(f32), q_dims: QMVDims, kv_rows: u32) Error!void {
    try ctx.check(c.nnz_dispatch_fused_norm_qkv_f16io(ctx.raw, wq, wk, wv, residual.ptr, q.raw(), k.raw(), v.raw(), norm_scale.ptr, q_dims, kv_rows));
}

// ---- Q4 family (transformer.zig:1895-2387) ---------------------------------

/// transformer.zig:1565 dispatchQMV's 4-bit form (the generic f32 path)
pub fn dispatchQ4MV(ctx: Ctx, w: *const QWeight, input: Buf(f32), output: Buf(f32), dims: QMVDims) Error!void {
    try ctx.check(c.nnz_dispatch_q4mv(ctx.raw, w, input.ptr, output.ptr, dims));
}

/// transformer.zig:1987 dispatchQ4MVf16ioResadd
pub fn dispatchQ4MVf16ioResadd(ctx: Ctx, w: *const QWeight, input: Buf(f16), residual: Buf(f32), dims: QMVDims) Error!void {
    try ctx.check(c.nnz_dispatch_q4mv_f16io_resadd(ctx.raw, w, input.raw(), residual.ptr, dims));
}

/// transformer.zig:2318 dispatchQ4FusedNormPairSiLUf16io
pub fn dispatchQ4FusedNormPairSiLUf16io(ctx: Ctx, w_gate: *const QWeight, w_up: *const QWeight, residual: Buf(f32), output: Buf(f16), norm_scale: Buf(f32), dims: QMVDims) Error!void {
    try ctx.check(c.nnz_dispatch_q4_fused_norm_pair_silu_f16io(ctx.raw, w_gate, w_up, residual.ptr, output.raw(), norm_scale.ptr, dims));
}

// ---- attention, norms, RoPE, KV, embedding (transformer.zig:667-1120) ------

/// transformer.zig:669 dispatchRMSNorm (out_dtype picks the pipeline variant)
pub fn dispatchRMSNorm(ctx: Ctx, input: Buf(f32), scale: Buf(f32), output: ?*anyopaque, out_dtype: c_int, bf16_trunc: bool, dims: RMSNormDims) Error!void {
    try ctx.check(c.nnz_dispatch_rms_norm(ctx.raw, input.ptr, scale.ptr, output, out_dtype, @intFromBool(bf16_trunc), dims));
}

/// transformer.zig:740 dispatchRoPE (in place)
pub fn dispatchRoPE(ctx: Ctx, data: ?*anyopaque, dtype: c_int, dims: RoPEDims) Error!void {
    try ctx.check(c.nnz_dispatch_rope(ctx.raw, data, dtype, dims));
}

/// transformer.zig:1030 dispatchGQAAttention (scratch: nnz_gqa_scratch_bytes)
pub fn dispatchGQAAttention(ctx: Ctx, q: ?*const anyopaque, q_dtype: c_int, k_cache: ?*const anyopaque, v_cache: ?*const anyopaque, kv_dtype: c_int, v_transposed: bool, output: ?*anyopaque, out_dtype: c_int, scratch: Buf(u8), dims: GQADims) Error!void {
    try ctx.check(c.nnz_dispatch_gqa_attention(ctx.raw, q, q_dtype, k_cache, v_cache, kv_dtype, @intFromBool(v_transposed), output, out_dtype, @ptrCast(scratch.ptr), scratch.len, -1, 0.0, dims));
}

/// transformer.zig:962 dispatchGQAAttentionFusedTG
pub fn dispatchGQAAttentionFusedTG(ctx: Ctx, q: Buf(f16), k_cache: Buf(f16), v_cache: Buf(f16), output: Buf(f16), k_raw: Buf(f16), v_raw: Buf(f16), q_norm: Buf(f32), k_norm: Buf(f32), scratch: Buf(u8), dims: GQAFusedDims) Error!void {
    try ctx.check(c.nnz_dispatch_gqa_attention_fused(ctx.raw, q.raw(), k_cache.raw(), v_cache.raw(), output.raw(), k_raw.raw(), v_raw.raw(), q_norm.ptr, k_norm.ptr, @ptrCast(scratch.ptr), scratch.len, dims));
}

/// transformer.zig:1072 dispatchEmbeddingLookup (1-bit table)
pub fn dispatchEmbeddingLookup(ctx: Ctx, token_ids: Buf(u32), w: *const QWeight, output: Buf(f32), dims: EmbedDims) Error!void {
    try ctx.check(c.nnz_dispatch_embedding_lookup(ctx.raw, token_ids.ptr, w.codes, w.scales, output.ptr, dims));
}

/// transformer.zig:1097 dispatchResidualAdd
pub fn dispatchResidualAdd(ctx: Ctx, residual: Buf(f32), addition: Buf(f32), count: u32) Error!void {
    try ctx.check(c.nnz_dispatch_residual_add(ctx.raw, residual.ptr, addition.ptr, count));
}

// ---- the decoder and its loop (model.zig, transformer.zig:2389-4135) -------

pub const ModelConfig = c.nnz_model_config;

/// Model(Config).init + forwardDecode + generate on the device.
pub const Model = struct {
    raw: *c.nnz_model,
    ctx: Ctx,

    pub fn init(ctx: Ctx, cfg: *const ModelConfig) Error!Model {
        var raw: ?*c.nnz_model = null;
        try ctx.check(c.nnz_model_create(ctx.raw, cfg, &raw));
        return .{ .raw = raw.?, .ctx = ctx };
    }

    pub fn deinit(self: Model) void {
        _ = c.nnz_model_destroy(self.raw);
    }

    /// Device pointer and size of one weight / cache tensor (NNZ_T_*).
    pub fn tensor(self: Model, id: c_int, layer: u32) Error![]u8 {
        var p: ?*anyopaque = null;
        var n: usize = 0;
        try self.ctx.check(c.nnz_model_tensor(self.raw, id, layer, &p, &n));
        return @as([*]u8, @ptrCast(p.?))[0..n];
    }

    /// forwardDecode (transformer.zig:2566); logits in NNZ_T_LOGITS.
    pub fn forwardDecode(self: Model, token_id: u32, position: u32) Error!void {
        try self.ctx.check(c.nnz_model_forward_decode(self.raw, token_id, position));
    }

    /// generate (transformer.zig:3942): greedy unless setSampling was called.
    pub fn generate(self: Model, prompt: []const u32, out_tokens: []u32) Error!u32 {
        var count: u32 = 0;
        try self.ctx.check(c.nnz_model_generate(self.raw, prompt.ptr, @intCast(prompt.len), @intCast(out_tokens.len), out_tokens.ptr, null, null, 1, &count));
        return count;
    }

    /// GenerateOpts.params (SamplingParams, transformer.zig:3652-3657).
    pub fn setSampling(self: Model, temperature: f32, top_k: u32, top_p: f32, seed: u64) Error!void {
        const p = c.nnz_sampling_params{ .temperature = temperature, .top_k = top_k, .top_p = top_p, .reserved = 0, .seed = seed };
        try self.ctx.check(c.nnz_model_set_sampling(self.raw, &p));
    }

    /// GenerateOpts.eos_ids (isEosToken, transformer.zig:4126).
    pub fn setEos(self: Model, ids: []const u32) Error!void {
        try self.ctx.check(c.nnz_model_set_eos(self.raw, ids.ptr, @intCast(ids.len)));
    }
};
