//! FFI declarations of libtpthip (`include/tpthip.h`).  NOT COMPILED HERE: the build image has
//! no Rust toolchain.  Layouts follow the C header field for field; every function returns an
//! `int` status (`TPT_OK` = 0, negative = error) and `tpt_last_error()` holds the calling
//! thread's last message.
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

pub const TPT_OK: c_int = 0;
pub const TPT_ERR_INVALID: c_int = -1;
pub const TPT_ERR_HIP: c_int = -2;
pub const TPT_ERR_IO: c_int = -3;
pub const TPT_ERR_FORMAT: c_int = -4;
pub const TPT_ERR_UNSUPPORTED: c_int = -5;
pub const TPT_ERR_CANCELLED: c_int = -6;
pub const TPT_ERR_STATE: c_int = -7;
pub const TPT_ERR_OOM: c_int = -8;

pub const TPT_TYPE_F32: c_int = 0;
pub const TPT_TYPE_F16: c_int = 1;

#[repr(C)]
pub struct tpt_engine {
    _opaque: [u8; 0],
}

/// ModelInfo (src-tauri/src/engine/mod.rs:85-92) as fixed-size C strings.
#[repr(C)]
pub struct tpt_model_info {
    pub name: [c_char; 256],
    pub path: [c_char; 1024],
    pub size_bytes: u64,
    pub backend: [c_char; 64],
}

/// InferenceParams (mod.rs:35-59) without the prompt text (the caller tokenizes), plus the
/// EOS id find_eos_token gives (candle_engine.rs:76-83) and the sampling seed.
#[repr(C)]
pub struct tpt_infer_params {
    pub max_tokens: u32,
    pub temperature: f32,
    pub top_p: f32,
    pub repeat_penalty: f32,
    pub eos_token_id: i64,
    pub seed: u64,
}

#[repr(C)]
#[derive(Default, Debug, Clone, Copy)]
pub struct tpt_infer_stats {
    pub prompt_tokens: u32,
    pub cached_prefix: u32,
    pub generated: u32,
    pub prefill_ms: f64,
    pub decode_ms: f64,
    pub ttft_ms: f64,
}

#[repr(C)]
#[derive(Default, Debug, Clone, Copy)]
pub struct tpt_model_desc {
    pub architecture: [c_char; 32],
    pub n_layers: c_int,
    pub n_heads: c_int,
    pub n_kv_heads: c_int,
    pub head_dim: c_int,
    pub embed: c_int,
    pub ffn: c_int,
    pub vocab: c_int,
    pub context_length: c_int,
    pub max_ctx: c_int,
    pub kv_type: c_int,
    pub rms_eps: f32,
    pub rope_base: f32,
    pub rope_scale: f32,
    pub weight_bytes: u64,
    pub decode_bytes_per_token: u64,
    pub type_q: c_int,
    pub type_k: c_int,
    pub type_v: c_int,
    pub type_o: c_int,
    pub type_gate: c_int,
    pub type_up: c_int,
    pub type_down: c_int,
    pub type_embd: c_int,
    pub type_out: c_int,
}

/// progress(user, done, total) after each uploaded tensor.
pub type tpt_progress_fn = Option<unsafe extern "C" fn(user: *mut c_void, done: u32, total: u32)>;
/// on_token(user, token_id, done): 0 continues, non-zero cancels (one done=1 event follows).
pub type tpt_token_fn =
    Option<unsafe extern "C" fn(user: *mut c_void, token_id: u32, done: c_int) -> c_int>;

extern "C" {
    pub fn tpt_last_error() -> *const c_char;
    pub fn tpt_version() -> c_int;

    pub fn tpt_model_inspect(gguf_path: *const c_char, out: *mut tpt_model_desc) -> c_int;

    pub fn tpt_engine_create(device: c_int, out: *mut *mut tpt_engine) -> c_int;
    pub fn tpt_engine_set_kv_type(e: *mut tpt_engine, kv_type: c_int) -> c_int;
    pub fn tpt_engine_destroy(e: *mut tpt_engine) -> c_int;
    pub fn tpt_engine_load(
        e: *mut tpt_engine,
        model_path: *const c_char,
        progress: tpt_progress_fn,
        user: *mut c_void,
        info_out: *mut tpt_model_info,
    ) -> c_int;
    pub fn tpt_engine_unload(e: *mut tpt_engine) -> c_int;
    pub fn tpt_engine_is_loaded(e: *const tpt_engine) -> c_int;
    pub fn tpt_engine_model_info(e: *const tpt_engine, info_out: *mut tpt_model_info) -> c_int;
    pub fn tpt_engine_infer(
        e: *mut tpt_engine,
        params: *const tpt_infer_params,
        prompt: *const u32,
        n_prompt: usize,
        on_token: tpt_token_fn,
        user: *mut c_void,
        stats: *mut tpt_infer_stats,
    ) -> c_int;
    pub fn tpt_common_prefix_len(a: *const u32, na: usize, b: *const u32, nb: usize) -> usize;
    pub fn tpt_engine_cached_prefix(
        e: *const tpt_engine,
        tokens: *const u32,
        n: usize,
        out: *mut usize,
    ) -> c_int;
    pub fn tpt_engine_reset_cache(e: *mut tpt_engine) -> c_int;
}

/// The calling thread's last error message.
pub fn last_error() -> String {
    // SAFETY: tpt_last_error returns a NUL-terminated thread-local string that lives until the
    // next failing call on this thread; it is copied out at once.
    unsafe { std::ffi::CStr::from_ptr(tpt_last_error()) }
        .to_string_lossy()
        .into_owned()
}
