//! The new body of ops.attentionEx for src/ops.zig (it replaces the body of the function at
//! src/ops.zig:562-590; the signature, AttnShape, q_block, the attentionScratch* functions and
//! ops.attention, which forwards here, stay as they are).  Add `const gpu = @import("gpu.zig");`
//! at the top of src/ops.zig.  The reference's own names in scope there are used as they are:
//! Pool, AttnShape, V, clock, profile.
//!
//! pool and scratch are accepted and unused: the GPU context owns its device memory and stream.
//! The call is synchronous, writes only each row's n_head * d output columns, and returns finite
//! results for any finite input (zwg_attention_ex recomputes an x3 result holding a non-finite
//! value on the fp32-MFMA kernel).  Not compiled in this repository: no Zig toolchain here.

pub fn attentionEx(pool: *Pool, q: []const f32, k: []const f32, v: []const f32, sh: AttnShape, scratch: []f32, out: []f32) void {
    _ = pool;
    _ = scratch;
    var t = clock.Timer.start();
    std.debug.assert(sh.d % V == 0 and sh.n_head % sh.n_head_kv == 0);
    const s = gpu.Shape{
        .n_q = sh.n_q,
        .n_kv = sh.n_kv,
        .n_head = sh.n_head,
        .n_head_kv = sh.n_head_kv,
        .d = sh.d,
        .q_stride = sh.q_stride,
        .kv_stride = sh.kv_stride,
        .out_stride = sh.out_stride,
        .kt_stride = sh.kt_stride orelse 0,
        .causal = @intFromBool(sh.causal),
    };
    const c = gpu.ctx();
    gpu.check(c, gpu.zwg_attention_ex(c, q.ptr, k.ptr, v.ptr, &s, out.ptr), "attention");
    if (profile.enabled) profile.attention += t.lap();
}
