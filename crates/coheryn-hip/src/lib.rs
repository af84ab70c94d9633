//! The engine's continuous-batching step on one MI355X.
//!
//! `HipModel` stands where `coheryn_engine::Model` stands for the scheduler
//! (crates/coheryn-api/src/scheduler/batching.rs:11-59): it owns the
//! HBM-resident weights, the paged KV pool and the step's workspaces, and
//! `HipModel::step_batch` is `Model::step_batch` (inference/batch.rs:64-116)
//! computed by the HIP kernels of libcohx.so.  `HipState` replaces
//! `GenerationState`: the library keeps the prompt cursor, the pending token,
//! the sampler and the sequence's KV pages; the host keeps a handle.
//!
//! The scheduler gains one impl beside its `impl BatchModel for Model`:
//!
//! ```ignore
//! impl BatchModel for coheryn_hip::HipModel {
//!     type State = coheryn_hip::HipState;
//!     fn compatible(a: &Self::State, b: &Self::State) -> bool { a.compatible(b) }
//!     fn wait(_: &mut Self::State, _: f64) {}
//!     fn cancellation(s: &Self::State) -> Cancellation { s.cancellation() }
//!     fn step(&self, states: &mut [&mut Self::State],
//!             yield_work: &mut coheryn_engine::multimodal::WorkYield<'_>)
//!         -> coheryn_engine::Result<coheryn_engine::inference::BatchStep> {
//!         self.step_batch(states, yield_work)
//!     }
//! }
//! ```
pub mod ffi;

use coheryn_engine::inference::BatchStep;
use coheryn_engine::multimodal::WorkYield;
use coheryn_engine::{Cancellation, Error, ErrorCode, Result};
use std::ffi::{CStr, CString};
use std::os::raw::{c_char, c_int, c_void};
use std::path::Path;

/// A library status as the engine's `Error` (error.rs:6-41 classes).
fn error(code: c_int, message: String) -> Error {
    match code {
        ffi::COHX_INVALID_REQUEST => Error::request(message),
        ffi::COHX_RESOURCE => Error::resource(message),
        ffi::COHX_CANCELLED => Error::new(ErrorCode::Cancelled, message),
        ffi::COHX_UNSUPPORTED => Error::new(ErrorCode::UnsupportedFeature, message),
        ffi::COHX_DEAD_END => Error::new(ErrorCode::ConstraintDeadEnd, message),
        ffi::COHX_DEVICE => Error::new(ErrorCode::Internal, message),
        _ => Error::invalid(message),
    }
}

fn check(ctx: *const ffi::cohx_ctx, code: c_int) -> Result<()> {
    if code == ffi::COHX_OK {
        return Ok(());
    }
    // SAFETY: the library returns a NUL-terminated string owned by `ctx`
    // that stays valid until the next call on it.
    let message = unsafe { CStr::from_ptr(ffi::cohx_last_error(ctx)) }.to_string_lossy().into_owned();
    Err(error(code, message))
}

/// GPU counterpart of `coheryn_engine::Model` for the Qwen2 graph (and, made
/// by `create_qwen35`, the Qwen3.5 hybrid graph).
pub struct HipModel {
    ctx: *mut ffi::cohx_ctx,
    desc: ffi::cohx_model_desc,
}

// SAFETY: the context is driven by one thread at a time; the scheduler's
// single compute permit (scheduler.rs:201) serializes every call.
unsafe impl Send for HipModel {}
unsafe impl Sync for HipModel {}

impl Drop for HipModel {
    fn drop(&mut self) {
        // SAFETY: `ctx` came from cohx_load_gguf / cohx_create_qwen35 and is
        // destroyed once; every HipState borrows the model, so none outlives it.
        unsafe { ffi::cohx_destroy(self.ctx) }
    }
}

impl HipModel {
    /// `Model::load` (inference.rs:238-297) from a GGUF file: the library
    /// parses and validates the file (the engine's acceptance rules,
    /// gguf.rs:304-496 and compat.rs:54-221), reads the end-of-generation ids
    /// and uploads every tensor into HBM.  `capacity` sets max_lanes,
    /// max_rows, max_seqs, max_context and kv_pages; zeros take the defaults.
    pub fn load(path: &Path, capacity: ffi::cohx_model_desc, device: i32) -> Result<Self> {
        use std::os::unix::ffi::OsStrExt;
        let path = CString::new(path.as_os_str().as_bytes()).map_err(|_| Error::request("path contains NUL"))?;
        let mut desc = capacity;
        let mut ctx = std::ptr::null_mut();
        let mut text = [0 as c_char; 512];
        // SAFETY: every pointer is valid for the call; `text` is writable for its length.
        let code = unsafe {
            ffi::cohx_load_gguf(path.as_ptr(), device, &mut desc, &mut ctx, text.as_mut_ptr(), text.len())
        };
        if code != ffi::COHX_OK {
            // SAFETY: the library NUL-terminates what it writes into `text`.
            let message = unsafe { CStr::from_ptr(text.as_ptr()) }.to_string_lossy().into_owned();
            return Err(error(code, message));
        }
        Ok(HipModel { ctx, desc })
    }

    /// `qwen35::Model::load` (qwen35/mod.rs:103-193): the context, then each
    /// safetensors tensor by name (config.rs:193-309): matrices BF16 with
    /// ne0 = columns and ne1 = rows, vectors F32 or BF16, conv1d.weight
    /// [C][1][K] as ne0 = K, ne1 = C.
    pub fn create_qwen35(desc: &ffi::cohx_qwen35_desc, tensors: &[(&str, u32, u64, u64, &[u8])], device: i32)
        -> Result<Self> {
        let mut ctx = std::ptr::null_mut();
        // SAFETY: `desc` and `ctx` are valid for the call.
        let code = unsafe { ffi::cohx_create_qwen35(desc, device, &mut ctx) };
        if code != ffi::COHX_OK {
            return Err(error(code, "the Qwen3.5 device context could not be created".into()));
        }
        let mut model = HipModel { ctx, desc: ffi::cohx_model_desc::default() };
        model.desc.vocabulary = desc.vocabulary;
        model.desc.max_lanes = desc.max_lanes;
        for (name, dtype, ne0, ne1, bytes) in tensors {
            let name = CString::new(*name).map_err(|_| Error::request("tensor name contains NUL"))?;
            // SAFETY: `bytes` is readable for its length during the call.
            check(model.ctx, unsafe {
                ffi::cohx_upload_tensor(model.ctx, name.as_ptr(), *dtype, *ne0, *ne1, bytes.as_ptr().cast(), bytes.len())
            })?;
        }
        // SAFETY: `ctx` is live.
        check(model.ctx, unsafe { ffi::cohx_finalize(model.ctx) })?;
        Ok(model)
    }

    /// The file's configuration, the capacities in force and the EOG ids.
    pub fn description(&self) -> &ffi::cohx_model_desc {
        &self.desc
    }

    /// `Model::begin_generation` (generation.rs:53-242) from prompt ids.
    /// `prior`, a finished state of this model, gives its KV rows to the new
    /// generation up to the longest common prefix (generation.rs:189-202).
    pub fn begin_generation(&self, prompt: &[u32], options: &ffi::cohx_gen_options, cancel: Cancellation,
                            prior: Option<HipState>) -> Result<HipState> {
        let mut state = std::ptr::null_mut();
        let prior_ptr = prior.as_ref().map_or(std::ptr::null_mut(), |p| p.state);
        // SAFETY: pointers are valid for the call; `prior` (if any) is owned
        // here and freed when it drops below, after the library has taken
        // over its pages.
        check(self.ctx, unsafe {
            ffi::cohx_gen_begin(self.ctx, prompt.as_ptr(), prompt.len() as u32, options, prior_ptr, &mut state)
        })?;
        drop(prior);
        Ok(HipState { state, cancel })
    }

    /// `Model::step_batch` (inference/batch.rs:64-116): one token per lane
    /// for 1..=max_lanes states.  A shared failure is returned (the library
    /// has copied it to every lane, batch.rs:98-105); a lane's own failure
    /// surfaces at its next `sample`.  `yield_work` runs while the device
    /// computes, so the scheduler can lend its compute permit
    /// (batching.rs:229-239); its Err fails the step as Cancelled with no lane
    /// advanced.  A lane's Cancellation is passed to the library before the
    /// launch and again at every poll.
    pub fn step_batch(&self, states: &mut [&mut HipState], yield_work: &mut WorkYield<'_>) -> Result<BatchStep> {
        struct Hook<'a, 'b> {
            yield_work: &'a mut WorkYield<'b>,
            lanes: Vec<(*mut ffi::cohx_gen, Cancellation)>,
        }
        unsafe extern "C" fn poll(user: *mut c_void) -> c_int {
            // SAFETY: `user` is the Hook below, alive for the whole call.
            let hook = unsafe { &mut *(user as *mut Hook<'_, '_>) };
            for (state, cancel) in &hook.lanes {
                if cancel.check().is_err() {
                    // SAFETY: the state is live; cohx_gen_cancel is an atomic store.
                    unsafe { ffi::cohx_gen_cancel(*state) }
                }
            }
            if (hook.yield_work)().is_err() { 1 } else { 0 }
        }
        for s in states.iter() {
            if s.cancel.check().is_err() {
                // SAFETY: the state is live.
                unsafe { ffi::cohx_gen_cancel(s.state) }
            }
        }
        let pointers: Vec<*mut ffi::cohx_gen> = states.iter().map(|s| s.state).collect();
        let mut hook = Hook { yield_work, lanes: states.iter().map(|s| (s.state, s.cancel.clone())).collect() };
        let mut out = ffi::cohx_batch_step::default();
        // SAFETY: `pointers` and `hook` outlive the call; the library calls
        // `poll` only during it.
        check(self.ctx, unsafe {
            ffi::cohx_step_batch_hooked(self.ctx, pointers.as_ptr(), pointers.len() as u32, &mut out, Some(poll),
                                        (&mut hook as *mut Hook<'_, '_>).cast())
        })?;
        Ok(BatchStep {
            width: out.width as usize,
            completed_tokens: out.completed_tokens as usize,
            matrix_tiles: out.matrix_tiles,
            matrix_bytes: out.matrix_bytes,
        })
    }
}

/// GPU counterpart of `GenerationState` (generation.rs:244-394).
pub struct HipState {
    state: *mut ffi::cohx_gen,
    cancel: Cancellation,
}

// SAFETY: a state moves between the scheduler's threads by value and is
// never used by two threads at once (docs/BATCHING.md:23); cohx_gen_cancel,
// the one call another thread may make, is an atomic store.
unsafe impl Send for HipState {}

impl Drop for HipState {
    fn drop(&mut self) {
        // SAFETY: the state is owned here and freed once.
        unsafe { ffi::cohx_gen_free(self.state) }
    }
}

impl HipState {
    /// `GenerationState::compatible` (generation.rs:271-275).
    pub fn compatible(&self, other: &HipState) -> bool {
        // SAFETY: both states are live.
        unsafe { ffi::cohx_gen_compatible(self.state, other.state) != 0 }
    }

    pub fn cancellation(&self) -> Cancellation {
        self.cancel.clone()
    }

    /// `GenerationState::sample` (generation.rs:319-394): the next token, or
    /// None once the generation has finished.
    pub fn sample(&mut self) -> Result<Option<u32>> {
        let mut token = -1i64;
        // SAFETY: the state is live and `token` writable.
        let code = unsafe { ffi::cohx_gen_sample(self.state, &mut token) };
        if code != ffi::COHX_OK {
            return Err(error(code, "generation failed".into()));
        }
        Ok(u32::try_from(token).ok())
    }

    pub fn needs_forward(&self) -> bool {
        // SAFETY: the state is live.
        unsafe { ffi::cohx_gen_needs_forward(self.state) != 0 }
    }

    pub fn is_finished(&self) -> bool {
        // SAFETY: the state is live.
        unsafe { ffi::cohx_gen_is_finished(self.state) != 0 }
    }

    /// The generated ids so far.
    pub fn tokens(&self) -> Vec<u32> {
        // SAFETY: a null buffer with cap 0 only asks for the count.
        let n = unsafe { ffi::cohx_gen_tokens(self.state, std::ptr::null_mut(), 0) };
        let mut out = vec![0u32; n as usize];
        // SAFETY: `out` holds `n` entries.
        unsafe { ffi::cohx_gen_tokens(self.state, out.as_mut_ptr(), n) };
        out
    }
}
