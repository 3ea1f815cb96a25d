//! Zig binding of libzwgpu's C ABI (include/zw_gpu.h): zwhisper's attention, its device-resident
//! KV caches, linear layers and encoder layer on an AMD MI355X.  Every function and type the
//! header declares, field for field and argument for argument.  Drop this file in as src/gpu.zig;
//! src/ops.zig's attentionEx then calls zwg_attention_ex (zig/ops_attention.zig), and build.zig
//! links the library (INTEGRATION.md).  Status codes: 0 ok, 2 error (zwg_last_error says why).
//! Not compiled in this repository: the build image has no Zig toolchain.
const std = @import("std");

pub const OK: c_int = 0;
pub const ERROR: c_int = 2;

// ---- context, shapes, plans (zw_gpu.h: zwg_ctx, zwg_attn_shape, zwg_batch, zwg_limits, zwg_plan_info)

pub const Ctx = opaque {};

/// Mirror of ops.AttnShape (src/ops.zig:477-492); kt_stride 0 stands for null (row-major K).
pub const Shape = extern struct {
    n_q: u64,
    n_kv: u64,
    n_head: u64,
    n_head_kv: u64,
    d: u64,
    q_stride: u64,
    kv_stride: u64,
    out_stride: u64,
    kt_stride: u64,
    causal: u32,
    reserved: u32 = 0,
};

pub const Batch = extern struct {
    n_batch: u64,
    q_bstride: u64,
    k_bstride: u64,
    v_bstride: u64,
    out_bstride: u64,
    n_kv_dev: ?[*]const i32, // per-item key counts in device memory, or null
};

pub const DENSE_X3: u32 = 0;
pub const DENSE_FP32: u32 = 1;

pub const Limits = extern struct {
    workspace_bytes: u64 = 0,
    dense_math: u32 = DENSE_X3,
    reserved: u32 = 0,
    staging_bytes: u64 = 0,
};

pub const PlanInfo = extern struct {
    kernel: u32,
    rows_per_unit: u32,
    chunk_len: u64,
    max_chunks: u64,
    grid_blocks: u64,
    workspace_bytes: u64,
};

pub extern "zwgpu" fn zwg_version() c_int;
pub extern "zwgpu" fn zwg_open(device: c_int, limits: ?*const Limits, out: *?*Ctx) c_int;
pub extern "zwgpu" fn zwg_close(ctx: ?*Ctx) void;
pub extern "zwgpu" fn zwg_last_error(ctx: ?*const Ctx) [*:0]const u8;
pub extern "zwgpu" fn zwg_set_stream(ctx: *Ctx, hip_stream: ?*anyopaque) c_int;
pub extern "zwgpu" fn zwg_get_stream(ctx: *const Ctx) ?*anyopaque;
pub extern "zwgpu" fn zwg_sync(ctx: *Ctx) c_int;
pub extern "zwgpu" fn zwg_set_dense_math(ctx: *Ctx, mode: u32) c_int;

// ---- attention

/// Drop-in for ops.attentionEx: host slices, synchronous.
pub extern "zwgpu" fn zwg_attention_ex(ctx: *Ctx, q: [*]const f32, k: [*]const f32, v: [*]const f32,
    shape: *const Shape, out: [*]f32) c_int;
/// Drop-in for ops.attention.
pub extern "zwgpu" fn zwg_attention(ctx: *Ctx, q: [*]const f32, k: [*]const f32, v: [*]const f32, n_q: u64,
    n_kv: u64, n_state: u64, n_head: u64, causal: c_int, out: [*]f32) c_int;
pub extern "zwgpu" fn zwg_attention_dev(ctx: *Ctx, q: [*]const f32, k: [*]const f32, v: [*]const f32,
    shape: *const Shape, out: [*]f32) c_int;
pub extern "zwgpu" fn zwg_attention_batch_dev(ctx: *Ctx, q: [*]const f32, k: [*]const f32, v: [*]const f32,
    shape: *const Shape, batch: *const Batch, out: [*]f32) c_int;
/// No context, no allocation: split partials in the library's static 64 MiB scratch per GPU.
pub const NOALLOC_SCRATCH_BYTES: u64 = 64 << 20;
pub extern "zwgpu" fn zwg_attention_batch_noalloc(q: [*]const f32, k: [*]const f32, v: [*]const f32,
    shape: *const Shape, batch: ?*const Batch, out: [*]f32, dense_math: u32, hip_stream: ?*anyopaque) c_int;
pub extern "zwgpu" fn zwg_plan(shape: *const Shape, batch: ?*const Batch, workspace_bytes: u64,
    out: *PlanInfo) c_int;
pub extern "zwgpu" fn zwg_check_shape(shape: *const Shape, msg: ?[*]u8, msg_len: usize) c_int;

// ---- device-resident KV caches

pub const Kv = opaque {};
pub const KV_ROW: u32 = 0; // k, v: [n_ctx][n_head_kv * d] (Whisper decoder)
pub const KV_KT: u32 = 1; // k: [n_head_kv][d][n_ctx], v: [n_ctx][n_head_kv * d] (Qwen2)
pub const KvDesc = extern struct {
    n_layer: u64,
    n_seq: u64,
    n_ctx: u64,
    n_head_kv: u64,
    d: u64,
    layout: u32,
    reserved: u32 = 0,
    rope_base: f64, // > 0: NeoX rotary positions applied on append; 0: none
};
pub const KvInfo = extern struct {
    k: [*]f32,
    v: [*]f32,
    layer_stride: u64,
    seq_stride: u64,
    kv_stride: u64,
    kt_stride: u64,
};
pub const ROWS_ON_HOST: u32 = 1;
pub extern "zwgpu" fn zwg_kv_create(ctx: *Ctx, desc: *const KvDesc, out: *?*Kv) c_int;
pub extern "zwgpu" fn zwg_kv_destroy(kv: ?*Kv) void;
pub extern "zwgpu" fn zwg_kv_get_info(kv: *const Kv, out: *KvInfo) c_int;
pub extern "zwgpu" fn zwg_kv_append(kv: *Kv, layer: u64, seq: u64, pos: u64, n: u64, k_rows: [*]const f32,
    v_rows: [*]const f32, q: ?[*]f32, n_head: u64, q_stride: u64, flags: u32) c_int;
pub extern "zwgpu" fn zwg_kv_append_batch(kv: *Kv, layer: u64, seq0: u64, n_seq: u64, pos_dev: [*]const i32,
    k_rows: [*]const f32, v_rows: [*]const f32, q: ?[*]f32, n_head: u64, q_stride: u64) c_int;
pub extern "zwgpu" fn zwg_kv_read(kv: *Kv, layer: u64, seq: u64, k_host: ?[*]f32, v_host: ?[*]f32) c_int;

// ---- linear layers (f16 and int8 block weights)

pub const W_F16: u32 = 1;
pub const W_Q8: u32 = 2;
pub const Q8W_FROM_HOST: u32 = 1;
pub const EPI_NONE: u32 = 0;
pub const EPI_GELU: u32 = 1;
pub const EPI_ADD: u32 = 2;
pub const Q8w = opaque {};
pub extern "zwgpu" fn zwg_linear(ctx: *Ctx, x: [*]const f32, m: u64, k: u64, w: *const anyopaque, w_type: u32,
    bias: ?[*]const f32, n: u64, out: [*]f32) c_int;
pub extern "zwgpu" fn zwg_linear_dev(ctx: *Ctx, x: [*]const f32, m: u64, k: u64, w: *const anyopaque, w_type: u32,
    bias: ?[*]const f32, n: u64, out: [*]f32) c_int;
pub extern "zwgpu" fn zwg_linear_epi_dev(ctx: *Ctx, x: [*]const f32, m: u64, k: u64, w: *const anyopaque,
    w_type: u32, bias: ?[*]const f32, n: u64, out: [*]f32, out_stride: u64, epilogue: u32) c_int;
pub extern "zwgpu" fn zwg_linear_q8(ctx: *Ctx, x: [*]const f32, m: u64, k: u64, q: [*]const i8,
    scales: [*]const f32, bias: ?[*]const f32, n: u64, out: [*]f32) c_int;
pub extern "zwgpu" fn zwg_linear_q8_dev(ctx: *Ctx, x: [*]const f32, m: u64, k: u64, q: [*]const i8,
    scales: [*]const f32, bias: ?[*]const f32, n: u64, out: [*]f32) c_int;
pub extern "zwgpu" fn zwg_q8w_create(ctx: *Ctx, q: [*]const i8, scales: [*]const f32, n: u64, k: u64, flags: u32,
    out: *?*Q8w) c_int;
pub extern "zwgpu" fn zwg_q8w_destroy(w: ?*Q8w) void;
pub extern "zwgpu" fn zwg_q8w_shape(w: *const Q8w, n: ?*u64, k: ?*u64) c_int;
pub extern "zwgpu" fn zwg_linear_q8w_dev(ctx: *Ctx, x: [*]const f32, m: u64, w: *const Q8w, bias: ?[*]const f32,
    out: [*]f32) c_int;
pub extern "zwgpu" fn zwg_linear_q8w_epi_dev(ctx: *Ctx, x: [*]const f32, m: u64, w: *const Q8w,
    bias: ?[*]const f32, out: [*]f32, epilogue: u32) c_int;
pub extern "zwgpu" fn zwg_linear_q8w_group_dev(ctx: *Ctx, x: [*]const f32, m: u64, n_w: u32,
    w: [*]const *const Q8w, bias: ?[*]const ?[*]const f32, out: [*]const [*]f32) c_int;
pub extern "zwgpu" fn zwg_linear_q8w_qkv_kv_dev(ctx: *Ctx, x: [*]const f32, m: u64, w: [*]const *const Q8w,
    bias: ?[*]const ?[*]const f32, q_out: [*]f32, kv: *Kv, layer: u64, seq0: u64, pos_dev: [*]const i32) c_int;

// ---- layer norm, GELU, add, a whole encoder layer

pub const EncLayer = extern struct {
    attn_ln_w: [*]const f32,
    attn_ln_b: [*]const f32,
    q_w: *const anyopaque,
    q_b: [*]const f32,
    k_w: *const anyopaque,
    v_w: *const anyopaque,
    v_b: [*]const f32,
    o_w: *const anyopaque,
    o_b: [*]const f32,
    mlp_ln_w: [*]const f32,
    mlp_ln_b: [*]const f32,
    mlp0_w: *const anyopaque,
    mlp0_b: [*]const f32,
    mlp1_w: *const anyopaque,
    mlp1_b: [*]const f32,
};
pub extern "zwgpu" fn zwg_layer_norm_dev(ctx: *Ctx, x: [*]const f32, m: u64, n: u64, w: [*]const f32,
    b: [*]const f32, eps: f32, out: [*]f32) c_int;
pub extern "zwgpu" fn zwg_gelu_dev(ctx: *Ctx, x: [*]f32, count: u64) c_int;
pub extern "zwgpu" fn zwg_add_dev(ctx: *Ctx, x: [*]f32, y: [*]const f32, count: u64) c_int;
pub extern "zwgpu" fn zwg_encoder_layer_scratch(n_rows: u64, n_state: u64) u64;
pub extern "zwgpu" fn zwg_encoder_layer_dev(ctx: *Ctx, x: [*]f32, n_windows: u64, n_ctx: u64, n_state: u64,
    n_head: u64, w: *const EncLayer, scratch: [*]f32) c_int;

// ---- the Whisper text decoder: setAudio and forward for windows decoded in lockstep

pub const DecLayer = extern struct {
    attn_ln_w: [*]const f32,
    attn_ln_b: [*]const f32,
    q_w: *const Q8w,
    q_b: ?[*]const f32,
    k_w: *const Q8w,
    v_w: *const Q8w,
    v_b: ?[*]const f32,
    o_w: *const Q8w,
    o_b: ?[*]const f32,
    cross_ln_w: [*]const f32,
    cross_ln_b: [*]const f32,
    cq_w: *const Q8w,
    cq_b: ?[*]const f32,
    ck_w: *const Q8w,
    cv_w: *const Q8w,
    cv_b: ?[*]const f32,
    co_w: *const Q8w,
    co_b: ?[*]const f32,
    mlp_ln_w: [*]const f32,
    mlp_ln_b: [*]const f32,
    mlp0_w: *const Q8w,
    mlp0_b: ?[*]const f32,
    mlp1_w: *const Q8w,
    mlp1_b: ?[*]const f32,
};
pub const Decoder = extern struct {
    n_vocab: u64,
    n_state: u64,
    n_head: u64,
    n_layer: u64,
    te: *const Q8w,
    pe: [*]const f32,
    ln_w: [*]const f32,
    ln_b: [*]const f32,
    layers: [*]const DecLayer,
    self_kv: *Kv,
    cross_kv: *Kv,
};
pub extern "zwgpu" fn zwg_decoder_set_audio_dev(ctx: *Ctx, dec: *const Decoder, enc: [*]const f32, n_windows: u64,
    seq0: u64) c_int;
pub extern "zwgpu" fn zwg_decoder_scratch(m: u64, n_state: u64) u64;
pub extern "zwgpu" fn zwg_decoder_step_dev(ctx: *Ctx, dec: *const Decoder, tokens: [*]const i32, pos: [*]const i32,
    m: u64, seq0: u64, logits: [*]f32, scratch: [*]f32) c_int;

// ---- Qwen2's norm, MLP gate and decode step

pub extern "zwgpu" fn zwg_rms_norm_dev(ctx: *Ctx, x: [*]const f32, m: u64, n: u64, w: [*]const f32, eps: f32,
    out: [*]f32) c_int;
pub extern "zwgpu" fn zwg_silu_mul_dev(ctx: *Ctx, gate: [*]f32, up: [*]const f32, count: u64) c_int;
pub const LlmLayer = extern struct {
    attn_norm: [*]const f32,
    wq: *const Q8w,
    bq: ?[*]const f32,
    wk: *const Q8w,
    bk: ?[*]const f32,
    wv: *const Q8w,
    bv: ?[*]const f32,
    wo: *const Q8w,
    ffn_norm: [*]const f32,
    w_gate: *const Q8w,
    w_up: *const Q8w,
    w_down: *const Q8w,
};
pub const Llm = extern struct {
    n_vocab: u64,
    n_embd: u64,
    n_head: u64,
    n_head_kv: u64,
    n_ff: u64,
    n_layer: u64,
    eps: f32,
    reserved: u32,
    embd: *const Q8w,
    output: *const Q8w,
    output_norm: [*]const f32,
    layers: [*]const LlmLayer,
    kv: *Kv,
};
pub extern "zwgpu" fn zwg_llm_scratch(m: u64, n_embd: u64, n_ff: u64) u64;
pub extern "zwgpu" fn zwg_llm_step_dev(ctx: *Ctx, lm: *const Llm, tokens: [*]const i32, pos: [*]const i32, m: u64,
    seq0: u64, logits: [*]f32, scratch: [*]f32) c_int;
pub extern "zwgpu" fn zwg_llm_forward_scratch(n: u64, n_embd: u64, n_ff: u64) u64;
pub extern "zwgpu" fn zwg_llm_forward_dev(ctx: *Ctx, lm: *const Llm, tokens: [*]const i32, n: u64, seq: u64,
    pos0: u64, logits: [*]f32, scratch: [*]f32) c_int;

// ---- the calling thread's context

/// One context per thread that calls into ops (the zw_* handles are per thread too,
/// src/capi.zig:3-4), opened on first use on device 0.
threadlocal var tls_ctx: ?*Ctx = null;

pub fn ctx() *Ctx {
    if (tls_ctx) |c| return c;
    var c: ?*Ctx = null;
    if (zwg_open(0, null, &c) != OK) std.debug.panic("zwg_open: {s}", .{zwg_last_error(null)});
    tls_ctx = c;
    return c.?;
}

/// ops' preconditions are asserts and its API is infallible: a failed call panics, as a failed
/// assert does in ReleaseSafe.
pub fn check(c: ?*Ctx, rc: c_int, what: []const u8) void {
    if (rc != OK) std.debug.panic("{s} on the GPU failed: {s}", .{ what, zwg_last_error(c) });
}
