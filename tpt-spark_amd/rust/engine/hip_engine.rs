// HipEngine -- `impl LlmEngine` over libtpthip (MI355X / gfx950).  Goes to
// src-tauri/src/engine/hip_engine.rs behind the `engine-hip` feature.
//
// NOT COMPILED HERE: the build image has no Rust toolchain.  Its calling pattern (progress
// trampoline over a caller-owned slot, cancel by a non-zero callback return, the done event
// after a cancel, calls from several OS threads) is exercised against the real library by
// tests/test_gpu_engine_ffi.py.
//
// Shape of the file follows the engine template of tpt_gpu_engine.rs:15-62; semantics follow
// CandleEngine (candle_engine.rs:124-334): tokenizer.json next to the GGUF, EOS from the
// tokenizer's special tokens, prompt truncation to context_length - max_tokens, greedy when
// temperature <= 0, repeat penalty per occurrence.  The library keeps the KV cache across calls
// (prefix reuse like WgpuEngine, wgpu_engine.rs:186-206) and the token loop on the device.

use crate::engine::{InferenceParams, LlmEngine, ModelInfo, TokenEvent};
use anyhow::{anyhow, bail, Result};
use std::ffi::{c_void, CStr, CString};
use std::os::raw::{c_char, c_int};
use std::panic::{catch_unwind, AssertUnwindSafe};
use std::path::Path;
use std::sync::Mutex;
use tokenizers::Tokenizer;
use tpt_hip_sys as ffi;

/// Owner of one `tpt_engine`.  The handle is only ever used while `raw`'s guard is held, so
/// `infer(&self)` gets the interior mutability the KV cache and scratch need without an
/// unsafe `&self -> &mut` cast.
struct Raw(*mut ffi::tpt_engine);
// SAFETY: the C engine has no thread affinity (every entry point selects its device), and all
// access goes through the Mutex below.
unsafe impl Send for Raw {}

pub struct HipEngine {
    raw: Mutex<Raw>,
    info: Option<ModelInfo>,
    tokenizer: Option<Tokenizer>,
    eos: u32,
}

impl HipEngine {
    /// Creates the engine on device 0, or None when no usable GPU is present -- the probe
    /// default_engine() uses to fall through to the next backend (as TptGpuEngine::gpu_available
    /// does, tpt_gpu_engine.rs:26-28).
    pub fn try_new() -> Option<Self> {
        let mut e: *mut ffi::tpt_engine = std::ptr::null_mut();
        // SAFETY: out-pointer to a local.
        if unsafe { ffi::tpt_engine_create(0, &mut e) } != ffi::TPT_OK || e.is_null() {
            return None;
        }
        Some(Self { raw: Mutex::new(Raw(e)), info: None, tokenizer: None, eos: 2 })
    }
}

impl Drop for HipEngine {
    fn drop(&mut self) {
        let raw = self.raw.get_mut().unwrap_or_else(|p| p.into_inner());
        // SAFETY: the handle came from tpt_engine_create and is destroyed once.
        unsafe { ffi::tpt_engine_destroy(raw.0) };
        raw.0 = std::ptr::null_mut();
    }
}

/// tokenizer.json next to the GGUF, or in a directory named after its stem (the search of
/// candle_engine.rs:48-73, restated here so that `engine-hip` needs no candle feature).
fn find_tokenizer(gguf_path: &Path) -> Result<Tokenizer> {
    let dir = gguf_path.parent().unwrap_or(Path::new("."));
    let stem = gguf_path.file_stem().and_then(|s| s.to_str()).unwrap_or("model");
    for p in [dir.join("tokenizer.json"), dir.join(stem).join("tokenizer.json")] {
        if p.exists() {
            return Tokenizer::from_file(&p).map_err(|e| anyhow!("tokenizer load failed: {e}"));
        }
    }
    bail!("tokenizer.json not found next to the GGUF file (expected {})",
          dir.join("tokenizer.json").display())
}

/// The EOS id: the first special token of these names the tokenizer knows, else 2 (the
/// candidates and default of candle_engine.rs:76-83).
fn find_eos_token(tok: &Tokenizer) -> u32 {
    ["<|eot_id|>", "<|end_of_text|>", "</s>", "<eos>", "[EOS]"]
        .iter()
        .find_map(|t| tok.token_to_id(t))
        .unwrap_or(2)
}

fn c_str(b: &[c_char]) -> String {
    // SAFETY: the library NUL-terminates every string field of tpt_model_info.
    unsafe { CStr::from_ptr(b.as_ptr()) }.to_string_lossy().into_owned()
}

/// The progress callback as the library calls it: `user` points at the caller's
/// `Option<&dyn Fn(u32, u32)>`, which lives on load()'s stack until tpt_engine_load returns.
unsafe extern "C" fn progress_tramp(user: *mut c_void, done: u32, total: u32) {
    let slot = &*(user as *const Option<&(dyn Fn(u32, u32) + Send + Sync)>);
    if let Some(f) = slot {
        // a panic must not unwind into C
        let _ = catch_unwind(AssertUnwindSafe(|| f(done, total)));
    }
}

struct InferCtx<'a> {
    tok: &'a Tokenizer,
    on_token: &'a mut dyn FnMut(TokenEvent) -> Result<()>,
    err: Option<anyhow::Error>,
}

/// The token callback: decode the id like CandleEngine (candle_engine.rs:299-302) and hand the
/// event to on_token.  An Err (the caller's cancel, commands.rs:288-292) or a panic returns 1,
/// which stops the run.  The library then still delivers one done event, which on_token gets
/// after a cancel too, its result ignored, as WgpuEngine does (wgpu_engine.rs:297-300).
unsafe extern "C" fn token_tramp(user: *mut c_void, id: u32, done: c_int) -> c_int {
    let c = &mut *(user as *mut InferCtx);
    let r = catch_unwind(AssertUnwindSafe(|| -> Result<()> {
        let token = if done != 0 {
            String::new()
        } else {
            c.tok.decode(&[id], true).map_err(|e| anyhow!("decode error: {e}"))?
        };
        (c.on_token)(TokenEvent { token, done: done != 0 })
    }));
    if c.err.is_some() {
        return 1; // already cancelled: only the done event can arrive here
    }
    match r {
        Ok(Ok(())) => 0,
        Ok(Err(e)) => {
            c.err = Some(e);
            1
        }
        Err(_) => {
            c.err = Some(anyhow!("token callback panicked"));
            1
        }
    }
}

impl LlmEngine for HipEngine {
    fn load(
        &mut self,
        model_path: &str,
        on_progress: Option<&(dyn Fn(u32, u32) + Send + Sync)>,
    ) -> Result<ModelInfo> {
        let tokenizer = find_tokenizer(Path::new(model_path))?;
        let eos = find_eos_token(&tokenizer);
        let path = CString::new(model_path)?;
        // SAFETY: a plain C struct of arrays and integers; all-zero is a valid value.
        let mut info: ffi::tpt_model_info = unsafe { std::mem::zeroed() };
        // The slot the trampoline reads; it outlives the FFI call below.
        let slot: Option<&(dyn Fn(u32, u32) + Send + Sync)> = on_progress;
        let (cb, user): (ffi::tpt_progress_fn, *mut c_void) = if slot.is_some() {
            (Some(progress_tramp), &slot as *const _ as *mut c_void)
        } else {
            (None, std::ptr::null_mut())
        };
        let guard = self.raw.get_mut().map_err(|_| anyhow!("engine mutex poisoned"))?;
        // SAFETY: handle from tpt_engine_create; path, slot and info outlive the call.
        let rc = unsafe { ffi::tpt_engine_load(guard.0, path.as_ptr(), cb, user, &mut info) };
        if rc != ffi::TPT_OK {
            self.info = None;
            self.tokenizer = None;
            bail!(ffi::last_error());
        }
        let mi = ModelInfo {
            name: c_str(&info.name),
            path: c_str(&info.path),
            size_bytes: info.size_bytes,
            backend: c_str(&info.backend), // "hip-gfx950"
        };
        self.tokenizer = Some(tokenizer);
        self.eos = eos;
        self.info = Some(mi.clone());
        Ok(mi)
    }

    fn unload(&mut self) -> Result<()> {
        let raw = self.raw.get_mut().map_err(|_| anyhow!("engine mutex poisoned"))?;
        // SAFETY: handle from tpt_engine_create.  Frees the model's HBM before returning.
        unsafe { ffi::tpt_engine_unload(raw.0) };
        self.info = None;
        self.tokenizer = None;
        Ok(())
    }

    fn is_loaded(&self) -> bool {
        self.info.is_some()
    }

    fn model_info(&self) -> Option<&ModelInfo> {
        self.info.as_ref()
    }

    fn infer(
        &self,
        params: &InferenceParams,
        on_token: &mut dyn FnMut(TokenEvent) -> Result<()>,
    ) -> Result<()> {
        let tok = self.tokenizer.as_ref().ok_or_else(|| anyhow!("no model loaded"))?;
        let ids: Vec<u32> = tok
            .encode(params.prompt.as_str(), true)
            .map_err(|e| anyhow!("tokenize error: {e}"))?
            .get_ids()
            .to_vec();
        let p = ffi::tpt_infer_params {
            max_tokens: params.max_tokens,
            temperature: params.temperature,
            top_p: params.top_p,
            repeat_penalty: params.repeat_penalty,
            eos_token_id: self.eos as i64,
            seed: 42, // LogitsProcessor::new(42, ..), candle_engine.rs:267
        };
        let mut ctx = InferCtx { tok, on_token, err: None };
        let mut st = ffi::tpt_infer_stats::default();
        // The guard stays alive across the FFI call: the engine's cache is this call's alone.
        let guard = self.raw.lock().map_err(|_| anyhow!("engine mutex poisoned"))?;
        // SAFETY: handle from tpt_engine_create; ids, p, ctx and st outlive the call; the
        // trampoline only touches ctx.
        let rc = unsafe {
            ffi::tpt_engine_infer(
                guard.0,
                &p,
                ids.as_ptr(),
                ids.len(),
                Some(token_tramp),
                &mut ctx as *mut InferCtx as *mut c_void,
                &mut st,
            )
        };
        drop(guard);
        if let Some(e) = ctx.err {
            return Err(e); // the caller's own error, e.g. "inference cancelled"
        }
        if rc != ffi::TPT_OK {
            bail!(ffi::last_error());
        }
        tracing::info!(
            "hip: prompt={} cached={} generated={} prefill={:.1}ms decode={:.1}ms",
            st.prompt_tokens, st.cached_prefix, st.generated, st.prefill_ms, st.decode_ms
        );
        Ok(())
    }
}
