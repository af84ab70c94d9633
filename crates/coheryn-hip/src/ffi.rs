//! Raw bindings of `include/cohx.h`, one declaration per exported entry point
//! and one `#[repr(C)]` struct per C struct, fields in the header's order.
//! `tests/test_rust_ffi.py` (in the library's repository) checks every
//! declaration here against the header: names, argument counts and types.
#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_int, c_void};

// Status codes (cohx.h; classes of crates/coheryn-engine/src/error.rs:6-41).
pub const COHX_OK: c_int = 0;
pub const COHX_INVALID_REQUEST: c_int = 1;
pub const COHX_INVALID_GGUF: c_int = 2;
pub const COHX_RESOURCE: c_int = 3;
pub const COHX_CANCELLED: c_int = 4;
pub const COHX_UNSUPPORTED: c_int = 5;
pub const COHX_DEAD_END: c_int = 6;
pub const COHX_DEVICE: c_int = 7;

// GGML dtypes (gguf.rs:104-128).
pub const COHX_F32: u32 = 0;
pub const COHX_F16: u32 = 1;
pub const COHX_Q4_0: u32 = 2;
pub const COHX_Q5_0: u32 = 6;
pub const COHX_Q8_0: u32 = 8;
pub const COHX_Q4_K: u32 = 12;
pub const COHX_Q6_K: u32 = 14;
pub const COHX_BF16: u32 = 30;
pub const COHX_MIXED: u32 = 0x100;

pub const COHX_PAGE: u32 = 16;
pub const COHX_AT_END: u32 = 0xFFFF_FFFF;
pub const COHX_SKIP_HEAD: u32 = 2;
pub const COHX_NO_TOKEN: u32 = 0xFFFF_FFFF;

pub const COHX_FINISH_NONE: u32 = 0;
pub const COHX_FINISH_STOP: u32 = 1;
pub const COHX_FINISH_LENGTH: u32 = 2;
pub const COHX_FINISH_CANCELLED: u32 = 3;

#[repr(C)]
pub struct cohx_ctx {
    _opaque: [u8; 0],
}

#[repr(C)]
pub struct cohx_gen {
    _opaque: [u8; 0],
}

#[repr(C)]
#[derive(Debug, Default, Clone, Copy)]
pub struct cohx_model_desc {
    pub layers: u32,
    pub hidden: u32,
    pub intermediate: u32,
    pub heads: u32,
    pub kv_heads: u32,
    pub head_dim: u32,
    pub vocabulary: u32,
    pub context: u32,
    pub rope_base: f32,
    pub norm_epsilon: f32,
    pub weight_dtype: u32,
    pub tied: u32,
    pub kv_dtype: u32,
    pub max_lanes: u32,
    pub max_rows: u32,
    pub max_seqs: u32,
    pub max_context: u32,
    pub kv_pages: u32,
    pub n_eog: u32,
    pub eog: [u32; 4],
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct cohx_lane {
    pub seq: u32,
    pub n_tokens: u32,
    pub tokens: *const u32,
    pub start_position: u32,
    pub want_logits: u32,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct cohx_batch {
    pub n_lanes: u32,
    pub lanes: *const cohx_lane,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct cohx_lane_out {
    pub status: i32,
    pub argmax: u32,
    pub logits: *mut f32,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct cohx_step_out {
    pub lanes: *mut cohx_lane_out,
    pub width: u32,
    pub rows: u32,
    pub matrix_bytes: u64,
    pub kv_bytes: u64,
    pub elapsed_ns: u64,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct cohx_step_hooks {
    pub yield_: Option<unsafe extern "C" fn(user: *mut c_void) -> c_int>,
    pub user: *mut c_void,
    pub cancel: *const u32,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct cohx_kernel_stat {
    pub name: *const c_char,
    pub launches: u64,
    pub total_ms: f64,
    pub bytes: f64,
    pub flops: f64,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct cohx_qwen35_desc {
    pub layers: u32,
    pub hidden: u32,
    pub intermediate: u32,
    pub vocabulary: u32,
    pub heads: u32,
    pub kv_heads: u32,
    pub head_dim: u32,
    pub linear_key_heads: u32,
    pub linear_value_heads: u32,
    pub linear_key_dim: u32,
    pub linear_value_dim: u32,
    pub conv_kernel: u32,
    pub rotary_dim: u32,
    pub context: u32,
    pub tied: u32,
    pub epsilon: f32,
    pub rope_base: f32,
    pub full_attention: [u8; 128],
    pub max_lanes: u32,
    pub max_rows: u32,
    pub max_seqs: u32,
    pub max_context: u32,
    pub n_eog: u32,
    pub eog: [u32; 4],
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct cohx_gen_options {
    pub max_tokens: u32,
    pub temperature: f32,
    pub top_k: u32,
    pub top_p: f32,
    pub seed: u64,
    pub repetition_penalty: f32,
    pub frequency_penalty: f32,
    pub presence_penalty: f32,
    pub n_stop_tokens: u32,
    pub stop_tokens: *const u32,
    pub context: u32,
}

#[repr(C)]
#[derive(Debug, Default, Clone, Copy)]
pub struct cohx_batch_step {
    pub width: u32,
    pub completed_tokens: u32,
    pub matrix_tiles: u64,
    pub matrix_bytes: u64,
}

pub type cohx_yield_fn = Option<unsafe extern "C" fn(user: *mut c_void) -> c_int>;

unsafe extern "C" {
    pub fn cohx_create(desc: *const cohx_model_desc, device: c_int, out: *mut *mut cohx_ctx) -> c_int;
    pub fn cohx_destroy(ctx: *mut cohx_ctx);
    pub fn cohx_last_error(ctx: *const cohx_ctx) -> *const c_char;
    pub fn cohx_load_gguf(
        path: *const c_char,
        device: c_int,
        desc: *mut cohx_model_desc,
        out: *mut *mut cohx_ctx,
        err: *mut c_char,
        err_cap: usize,
    ) -> c_int;
    pub fn cohx_gguf_inspect(path: *const c_char, desc: *mut cohx_model_desc, err: *mut c_char, err_cap: usize)
        -> c_int;
    pub fn cohx_upload_tensor(
        ctx: *mut cohx_ctx,
        name: *const c_char,
        dtype: u32,
        ne0: u64,
        ne1: u64,
        data: *const c_void,
        bytes: usize,
    ) -> c_int;
    pub fn cohx_finalize(ctx: *mut cohx_ctx) -> c_int;

    pub fn cohx_seq_alloc(ctx: *mut cohx_ctx, capacity: u32, seq: *mut u32) -> c_int;
    pub fn cohx_seq_fork(ctx: *mut cohx_ctx, src: u32, rows: u32, capacity: u32, seq: *mut u32) -> c_int;
    pub fn cohx_seq_free(ctx: *mut cohx_ctx, seq: u32) -> c_int;
    pub fn cohx_seq_truncate(ctx: *mut cohx_ctx, seq: u32, rows: u32) -> c_int;
    pub fn cohx_seq_length(ctx: *const cohx_ctx, seq: u32, rows: *mut u32) -> c_int;
    pub fn cohx_seq_pages(ctx: *const cohx_ctx, seq: u32, out: *mut i32, cap: u32) -> u32;
    pub fn cohx_seq_read_kv(ctx: *mut cohx_ctx, seq: u32, layer: u32, values: c_int, out: *mut f32) -> c_int;
    pub fn cohx_seq_read_kv_rows(
        ctx: *mut cohx_ctx,
        seq: u32,
        layer: u32,
        values: c_int,
        first: u32,
        count: u32,
        out: *mut f32,
    ) -> c_int;
    pub fn cohx_seq_fill_synthetic(ctx: *mut cohx_ctx, seq: u32, rows: u32, seed: u64, stream: u32) -> c_int;

    pub fn cohx_step(ctx: *mut cohx_ctx, batch: *const cohx_batch, out: *mut cohx_step_out) -> c_int;
    pub fn cohx_step_hooked(
        ctx: *mut cohx_ctx,
        batch: *const cohx_batch,
        out: *mut cohx_step_out,
        hooks: *const cohx_step_hooks,
    ) -> c_int;
    pub fn cohx_step_noalloc(ctx: *mut cohx_ctx, batch: *const cohx_batch, out: *mut cohx_step_out) -> c_int;
    pub fn cohx_pack(
        ctx: *mut cohx_ctx,
        batch: *const cohx_batch,
        cu_seqlens: *mut u32,
        positions: *mut u32,
        slots: *mut i64,
        lanes: *mut u32,
    ) -> c_int;
    pub fn cohx_matvec(
        ctx: *mut cohx_ctx,
        dtype: u32,
        rows: u32,
        k: u32,
        weights: *const c_void,
        bytes: usize,
        n: u32,
        inputs: *const f32,
        out: *mut f32,
        act_bytes: *mut u8,
        decoded: *mut f32,
        status: *mut i32,
    ) -> c_int;
    pub fn cohx_profile(ctx: *mut cohx_ctx, enable: c_int) -> c_int;
    pub fn cohx_profile_read(ctx: *const cohx_ctx, out: *mut cohx_kernel_stat, cap: u32) -> u32;

    pub fn cohx_create_qwen35(desc: *const cohx_qwen35_desc, device: c_int, out: *mut *mut cohx_ctx) -> c_int;

    pub fn cohx_gen_begin(
        ctx: *mut cohx_ctx,
        prompt: *const u32,
        n_prompt: u32,
        options: *const cohx_gen_options,
        prior: *mut cohx_gen,
        out: *mut *mut cohx_gen,
    ) -> c_int;
    pub fn cohx_step_batch(ctx: *mut cohx_ctx, states: *const *mut cohx_gen, n: u32, out: *mut cohx_batch_step)
        -> c_int;
    pub fn cohx_step_batch_hooked(
        ctx: *mut cohx_ctx,
        states: *const *mut cohx_gen,
        n: u32,
        out: *mut cohx_batch_step,
        yield_: cohx_yield_fn,
        user: *mut c_void,
    ) -> c_int;
    pub fn cohx_step_generation(ctx: *mut cohx_ctx, state: *mut cohx_gen) -> c_int;
    pub fn cohx_gen_sample(state: *mut cohx_gen, token: *mut i64) -> c_int;
    pub fn cohx_gen_needs_forward(state: *const cohx_gen) -> c_int;
    pub fn cohx_gen_is_finished(state: *const cohx_gen) -> c_int;
    pub fn cohx_gen_is_prefilling(state: *const cohx_gen) -> c_int;
    pub fn cohx_gen_finish_reason(state: *const cohx_gen) -> u32;
    pub fn cohx_gen_tokens(state: *const cohx_gen, out: *mut u32, cap: u32) -> u32;
    pub fn cohx_gen_cancel(state: *mut cohx_gen);
    pub fn cohx_gen_compatible(a: *const cohx_gen, b: *const cohx_gen) -> c_int;
    pub fn cohx_gen_free(state: *mut cohx_gen);
}
