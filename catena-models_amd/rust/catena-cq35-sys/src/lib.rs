//! Raw declarations of `include/cq35.h` (ABI version 3) and thin owning
//! wrappers, for catena-models' Rust host. The host replaces its three
//! `Artifact::exec_values` call sites for the Qwen artifact
//! (src/model.rs:248-258 `qwen3.init`, 260-328 `qwen3`, 209-246
//! `qwen3.copy-buffer`) with `Model::session`, `Session::step` and
//! `Session::copy`; everything else (ModelConfig, weight_specs order, the
//! range checks before each call) stays on the Rust side.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int, c_void, CStr, CString};
use std::marker::PhantomData;
use std::os::unix::ffi::OsStrExt;
use std::path::Path;

pub const CQ35_ABI_VERSION: c_int = 3;
pub const CQ35_OK: c_int = 0;
pub const CQ35_EINVAL: c_int = -1;
pub const CQ35_ERANGE: c_int = -2;
pub const CQ35_EDEVICE: c_int = -3;
pub const CQ35_EUNSUPPORTED: c_int = -4;
pub const CQ35_EPOISONED: c_int = -5;
pub const CQ35_MATRIX_PROJECTIONS: c_int = 1;
pub const CQ35_MATRIX_EXPERTS: c_int = 2;
pub const CQ35_MATRIX_ATTENTION: c_int = 4;
pub const CQ35_SPLIT_KEYS_DEFAULT: i64 = 8192;

/// The ModelConfig fields the token loop reads (src/spec.rs:33-62), in the
/// layout of `cq35_config`.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq)]
pub struct cq35_config {
    pub moe: i32,
    pub vocab: i32,
    pub hidden: i32,
    pub intermediate: i32,
    pub layers: i32,
    pub q_heads: i32,
    pub kv_heads: i32,
    pub head_dim: i32,
    pub rope_dim: i32,
    pub eps: f32,
    pub theta: f32,
    pub experts: i32,
    pub top_k: i32,
    pub shared_intermediate: i32,
    pub full_interval: i32,
    pub key_heads: i32,
    pub key_dim: i32,
    pub value_heads: i32,
    pub value_dim: i32,
    pub tied: i32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct cq35_tensor_info {
    pub dtype: i32,
    pub rows: i64,
    pub cols: i64,
    pub bytes: i64,
}

#[repr(C)]
pub struct cq35_model {
    _p: [u8; 0],
}
#[repr(C)]
pub struct cq35_session {
    _p: [u8; 0],
}

extern "C" {
    pub fn cq35_last_error() -> *const c_char;
    pub fn cq35_abi_version() -> c_int;
    pub fn cq35_config_validate(cfg: *const cq35_config) -> c_int;
    pub fn cq35_weight_count(cfg: *const cq35_config, count: *mut i64) -> c_int;
    pub fn cq35_weight_info(cfg: *const cq35_config, index: i64, info: *mut cq35_tensor_info) -> c_int;
    pub fn cq35_model_create(cfg: *const cq35_config, weights: *const *const c_void, on_device: c_int,
                             out: *mut *mut cq35_model) -> c_int;
    pub fn cq35_gguf_config(path: *const c_char, out: *mut cq35_config) -> c_int;
    pub fn cq35_gguf_validate(path: *const c_char, cfg: *const cq35_config) -> c_int;
    pub fn cq35_model_load_gguf(path: *const c_char, out: *mut *mut cq35_model) -> c_int;
    pub fn cq35_model_free(model: *mut cq35_model) -> c_int;
    pub fn cq35_model_config(model: *const cq35_model, out: *mut cq35_config) -> c_int;
    pub fn cq35_session_init(model: *mut cq35_model, capacity: i64, out: *mut *mut cq35_session) -> c_int;
    pub fn cq35_session_free(session: *mut cq35_session) -> c_int;
    pub fn cq35_step(session: *mut cq35_session, tokens: *const u64, n: i64, start: i64, capacity: i64,
                     next_token: *mut u64, logits: *mut u16) -> c_int;
    pub fn cq35_step_batch(sessions: *const *mut cq35_session, tokens: *const u64, starts: *const i64,
                           count: i64, next_tokens: *mut u64, logits: *mut u16) -> c_int;
    pub fn cq35_step_static(model: *const cq35_model, state: *mut u16, capacity: i64, token: u64, start: i64,
                            stream: *mut c_void, next_token: *mut u64, logits: *mut u16) -> c_int;
    pub fn cq35_session_copy(src: *const cq35_session, out: *mut *mut cq35_session) -> c_int;
    pub fn cq35_session_state_bytes(session: *const cq35_session, which: c_int, bytes: *mut i64) -> c_int;
    pub fn cq35_session_export_state(session: *const cq35_session, which: c_int, dst: *mut c_void,
                                     bytes: i64) -> c_int;
    pub fn cq35_session_import_state(session: *mut cq35_session, which: c_int, src: *const c_void,
                                     bytes: i64) -> c_int;
    pub fn cq35_session_set_persistent(session: *mut cq35_session, enabled: c_int) -> c_int;
    pub fn cq35_session_set_attention_split(session: *mut cq35_session, keys: i64) -> c_int;
    pub fn cq35_session_set_matrix_prefill(session: *mut cq35_session, components: c_int) -> c_int;
    pub fn cq35_session_set_matrix_decode(session: *mut cq35_session, enabled: c_int) -> c_int;
}

/// `Ok(())` for CQ35_OK, else the code with the library's message for this thread.
pub fn check(rc: c_int) -> anyhow::Result<()> {
    if rc == CQ35_OK {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(cq35_last_error()) }.to_string_lossy().into_owned();
    anyhow::bail!("cq35 error {rc}: {msg}")
}

/// Weights placed in HBM once (the reference keeps zero-copy host views,
/// src/checkpoint.rs:197-231). `Send` but not `Sync`: the model may move to
/// another thread, and its sessions borrow it, so it outlives them.
pub struct Model(*mut cq35_model);
unsafe impl Send for Model {}

impl Model {
    /// `weights[i]`: host pointer of tensor i in weight_specs order (src/spec.rs:443-712).
    pub fn from_host(cfg: &cq35_config, weights: &[*const c_void]) -> anyhow::Result<Self> {
        anyhow::ensure!(unsafe { cq35_abi_version() } == CQ35_ABI_VERSION, "libcq35 ABI version mismatch");
        let mut n = 0i64;
        check(unsafe { cq35_weight_count(cfg, &mut n) })?;
        anyhow::ensure!(weights.len() as i64 == n, "expected {n} weights, got {}", weights.len());
        let mut m = std::ptr::null_mut();
        check(unsafe { cq35_model_create(cfg, weights.as_ptr(), 0, &mut m) })?;
        Ok(Model(m))
    }

    /// Model::load_gguf (src/model.rs:43, 81-153) for qwen35 / qwen35moe files.
    pub fn load_gguf(path: &Path) -> anyhow::Result<Self> {
        let c = CString::new(path.as_os_str().as_bytes())?;
        let mut m = std::ptr::null_mut();
        check(unsafe { cq35_model_load_gguf(c.as_ptr(), &mut m) })?;
        Ok(Model(m))
    }

    pub fn config(&self) -> anyhow::Result<cq35_config> {
        let mut c = cq35_config::default();
        check(unsafe { cq35_model_config(self.0, &mut c) })?;
        Ok(c)
    }

    /// `qwen3.init(capacity)` (src/model.rs:248-258). The session borrows
    /// the model (as the reference's `Session<'a>` borrows `&'a Model`,
    /// src/model.rs:421-427): the weights cannot be freed while it lives.
    pub fn session(&self, capacity: i64) -> anyhow::Result<Session<'_>> {
        let vocab = self.config()?.vocab as usize;
        let mut s = std::ptr::null_mut();
        check(unsafe { cq35_session_init(self.0, capacity, &mut s) })?;
        Ok(Session { raw: s, capacity, vocab, _model: PhantomData })
    }
}

impl Drop for Model {
    fn drop(&mut self) {
        unsafe { cq35_model_free(self.0) };
    }
}

/// The opaque session state (BF16 cache, F32 workspace). One caller at a
/// time (`&mut self`); after a failed step the state is gone
/// (CQ35_EPOISONED), as the reference drops its state when exec fails
/// (src/model.rs:711-730). Distinct sessions may step on distinct threads.
pub struct Session<'m> {
    raw: *mut cq35_session,
    capacity: i64,
    vocab: usize,
    _model: PhantomData<&'m Model>,
}
unsafe impl Send for Session<'_> {}

impl<'m> Session<'m> {
    /// `qwen3(tokens, state, capacity, start, weights...)` (src/model.rs:260-328):
    /// the tokens at positions start..start+n, the greedy next token, and
    /// the last position's BF16 logits when `logits` is given (vocab entries).
    pub fn step(&mut self, tokens: &[u64], start: i64, logits: Option<&mut [u16]>) -> anyhow::Result<u64> {
        let mut next = 0u64;
        if let Some(l) = logits.as_deref() {
            anyhow::ensure!(l.len() >= self.vocab, "logits buffer holds {} entries, vocab is {}", l.len(), self.vocab);
        }
        let lp = logits.map_or(std::ptr::null_mut(), |l| l.as_mut_ptr());
        check(unsafe {
            cq35_step(self.raw, tokens.as_ptr(), tokens.len() as i64, start, self.capacity, &mut next, lp)
        })?;
        Ok(next)
    }

    /// `qwen3.copy-buffer(-16)` over the whole state (src/model.rs:209-246).
    pub fn copy(&self) -> anyhow::Result<Session<'m>> {
        let mut s = std::ptr::null_mut();
        check(unsafe { cq35_session_copy(self.raw, &mut s) })?;
        Ok(Session { raw: s, capacity: self.capacity, vocab: self.vocab, _model: PhantomData })
    }

    /// InferenceOptions::wmma_prefill (src/catena.rs:12-26): CQ35_MATRIX_* bits.
    pub fn set_matrix_prefill(&mut self, components: c_int) -> anyhow::Result<()> {
        check(unsafe { cq35_session_set_matrix_prefill(self.raw, components) })
    }

    /// Matrix-core products in `step_batch` when every session of the batch
    /// sets this (tolerance-level; no reference counterpart).
    pub fn set_matrix_decode(&mut self, enabled: bool) -> anyhow::Result<()> {
        check(unsafe { cq35_session_set_matrix_decode(self.raw, enabled as c_int) })
    }

    pub fn raw(&self) -> *mut cq35_session {
        self.raw
    }
}

impl Drop for Session<'_> {
    fn drop(&mut self) {
        unsafe { cq35_session_free(self.raw) };
    }
}

/// One decode step for each session (a serving round; the reference steps
/// them one after another, src/server/engine.rs:143-207). With `logits`,
/// session i's BF16 logits land in `logits[i * vocab ..]`.
pub fn step_batch(sessions: &mut [&mut Session<'_>], tokens: &[u64], starts: &[i64],
                  logits: Option<&mut [u16]>) -> anyhow::Result<Vec<u64>> {
    anyhow::ensure!(sessions.len() == tokens.len() && tokens.len() == starts.len(), "one token and start per session");
    if let Some(l) = logits.as_deref() {
        let need = sessions.iter().map(|s| s.vocab).sum::<usize>();
        anyhow::ensure!(sessions.iter().all(|s| s.vocab == sessions[0].vocab), "sessions of different vocabularies");
        anyhow::ensure!(l.len() >= need, "logits buffer holds {} entries, {} sessions need {need}", l.len(),
                        sessions.len());
    }
    let raw: Vec<*mut cq35_session> = sessions.iter().map(|s| s.raw).collect();
    let mut next = vec![0u64; raw.len()];
    let lp = logits.map_or(std::ptr::null_mut(), |l| l.as_mut_ptr());
    check(unsafe { cq35_step_batch(raw.as_ptr(), tokens.as_ptr(), starts.as_ptr(), raw.len() as i64, next.as_mut_ptr(), lp) })?;
    Ok(next)
}
