//! HardShell on AMD Instinct MI355X (gfx950): the integer GPT-2 of `hardshell` on hand-written
//! int8 MFMA kernels, bit for bit equal to the CPU reference.
//!
//! This crate is the safe face of `libhardshell_hip.so` (built by `taco_amd/build.py` with
//! `hipcc --offload-arch=gfx950`; `build.rs` links it). Its types mirror the public API of
//! `hardshell-cuda` one for one, so `taco` drives them the way it drives the CUDA backend:
//!
//! - [`HipDevice`]: one GPU (`CudaDevice`, `crates/hardshell-cuda/src/device.rs:21-74`).
//! - [`HipModel`]: a model file in GPU memory (`CudaModel`, `model.rs:231-398`).
//! - [`HipBatch`]: many independent sessions and prefill of many positions per pass
//!   (`CudaBatch`, `batch.rs:228-498`, `batch/stream.rs`, `batch/mixed.rs`).
//! - [`HipSession`]: one session (`CudaSession`, `session.rs:20-91`).
//!
//! Every call is synchronous. The handles use the calling thread's device, so none of these
//! types is `Send` (raw pointers inside), as with `CudaDevice`.

mod ffi;

use core::ffi::{c_char, c_void};
use std::ffi::CStr;

use hardshell::gpt2::Overlap;
use hardshell::{ModelHash, TokenId};

pub use ffi::{HS_MIX_NONE, HS_MIX_PLAIN};

/// A result with the error of this crate.
pub type Result<T> = std::result::Result<T, Error>;

/// An error of the HIP backend: the variants of `hardshell_cuda::Error`
/// (`crates/hardshell-cuda/src/error.rs:9-51`), each a thing a caller can act on.
#[derive(Debug, thiserror::Error)]
#[non_exhaustive]
pub enum Error {
    /// No HIP runtime or no device. The caller can use another backend.
    #[error("no HIP device: {reason}")]
    NoDevice {
        /// What is missing.
        reason: String,
    },
    /// A HIP runtime call or a kernel launch failed.
    #[error("{call} failed: {reason} ({code})")]
    Hip {
        /// The entry point that failed.
        call: &'static str,
        /// The HIP error code.
        code: i32,
        /// The message of the library.
        reason: String,
    },
    /// The device, the model or the request has a shape that the kernels do not support.
    #[error("not supported: {reason}")]
    Unsupported {
        /// Why.
        reason: String,
    },
    /// The model file or a token is not valid: the kind is the `hs_model_error` value, in the
    /// order of the variants of `hardshell::Error`.
    #[error("model error {kind}: {reason}")]
    Model {
        /// The `hs_model_error` value.
        kind: i32,
        /// The message of the library.
        reason: String,
    },
    /// A slot index is not in the batch.
    #[error("slot {slot} is not valid in a batch of {slots} slots")]
    BadSlot {
        /// The slot.
        slot: usize,
        /// The number of slots in the batch.
        slots: usize,
    },
    /// The lengths of two arguments do not agree.
    #[error("length mismatch: expected {expected}, found {found}")]
    LengthMismatch {
        /// The length that was expected.
        expected: usize,
        /// The length that was found.
        found: usize,
    },
}

fn last_message() -> String {
    // SAFETY: the library returns a NUL-terminated string owned by the calling thread.
    unsafe { CStr::from_ptr(ffi::hs_last_error_message()) }.to_string_lossy().into_owned()
}

/// The error of a status other than `HS_OK` (the message and code of the failure are the
/// calling thread's).
fn check(call: &'static str, status: i32) -> Result<()> {
    if status == ffi::Status::Ok as i32 {
        return Ok(());
    }
    // SAFETY: plain reads of the thread's error state.
    let code = unsafe { ffi::hs_last_error_code() };
    let reason = last_message();
    Err(match status {
        s if s == ffi::Status::NoDevice as i32 => Error::NoDevice { reason },
        s if s == ffi::Status::Unsupported as i32 => Error::Unsupported { reason },
        s if s == ffi::Status::ModelError as i32 => Error::Model { kind: code, reason },
        s if s == ffi::Status::BadSlot as i32 => Error::Unsupported { reason },
        s if s == ffi::Status::LengthMismatch as i32 => Error::Unsupported { reason },
        _ => Error::Hip { call, code, reason },
    })
}

/// A question to the coder op (`hardshell_cuda::CoderQuery`).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
#[non_exhaustive]
pub enum CoderQuery {
    /// The interval of this token (the encoder).
    Encode(TokenId),
    /// The symbol whose interval holds this target, `target < 2^freq_bits` (the decoder).
    Decode(u64),
}

/// The interval of one symbol in `taco_coder::FreqTable::from_weights`
/// (`hardshell_cuda::CoderInterval`).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub struct CoderInterval {
    /// The symbol.
    pub symbol: TokenId,
    /// The sum of the frequencies of the lower symbols.
    pub start: u64,
    /// The frequency of the symbol, at least 1.
    pub freq: u64,
    /// The symbol is the last symbol of the table.
    pub is_last: bool,
}

/// The table of one input of the mixed coder op (`hardshell_cuda::MixInput`).
#[derive(Clone, Copy, Debug, PartialEq, Eq, Hash)]
#[non_exhaustive]
pub enum MixInput {
    /// The table of GPT-2 alone.
    Plain,
    /// The mixer table with this prediction of the match model.
    Mixed(Option<TokenId>),
}

/// The statistics of one input's weights for the host mixer (`hardshell_cuda::MixStats`).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub struct MixStats {
    /// `sum(w)`.
    pub total: u64,
    /// `w[p]`.
    pub predicted: u64,
    /// The token of the largest weight (the lowest id on a tie, token 0 if every weight is 0).
    pub top: TokenId,
}

/// One GPU with the kernels loaded (`hardshell_cuda::CudaDevice`).
pub struct HipDevice {
    raw: *mut ffi::hs_device,
    name: String,
}

impl std::fmt::Debug for HipDevice {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        f.debug_struct("HipDevice").field("name", &self.name).finish_non_exhaustive()
    }
}

impl HipDevice {
    /// Opens the GPU `ordinal`.
    ///
    /// # Errors
    /// [`Error::NoDevice`] without a HIP runtime or device; [`Error::Unsupported`] for a GPU
    /// that is not gfx950.
    pub fn open(ordinal: usize) -> Result<Self> {
        let ordinal = i32::try_from(ordinal).map_err(|_| Error::NoDevice { reason: "ordinal".to_owned() })?;
        let mut raw = core::ptr::null_mut();
        // SAFETY: `raw` is a valid out-pointer.
        check("hs_device_open", unsafe { ffi::hs_device_open(ordinal, &mut raw) })?;
        let mut buf = [0 as c_char; 256];
        // SAFETY: the buffer holds `buf.len()` bytes.
        check("hs_device_name", unsafe { ffi::hs_device_name(raw, buf.as_mut_ptr(), buf.len()) })?;
        // SAFETY: the library wrote a NUL-terminated name into the buffer.
        let name = unsafe { CStr::from_ptr(buf.as_ptr()) }.to_string_lossy().into_owned();
        Ok(Self { raw, name })
    }

    /// The device name.
    #[must_use]
    pub fn name(&self) -> &str {
        &self.name
    }

    /// `(free, total)` bytes of device memory.
    ///
    /// # Errors
    /// [`Error::Hip`] if the runtime call fails.
    pub fn memory(&self) -> Result<(usize, usize)> {
        let (mut free, mut total) = (0usize, 0usize);
        // SAFETY: valid out-pointers.
        check("hs_device_memory", unsafe { ffi::hs_device_memory(self.raw, &mut free, &mut total) })?;
        Ok((free, total))
    }

    /// The main kernels with their registers, private (spill) bytes and static LDS bytes.
    ///
    /// # Errors
    /// [`Error::Hip`] if an attribute query fails.
    pub fn kernel_resources(&self) -> Result<Vec<(String, i32, i32, i32)>> {
        const CAP: usize = 64;
        let mut names = vec![0 as c_char; 64 * CAP];
        let (mut regs, mut private, mut lds) = (vec![0i32; CAP], vec![0i32; CAP], vec![0i32; CAP]);
        let mut count = 0usize;
        // SAFETY: every array holds CAP entries (names: 64-byte slots).
        check("hs_device_kernel_resources", unsafe {
            ffi::hs_device_kernel_resources(
                self.raw,
                names.as_mut_ptr(),
                regs.as_mut_ptr(),
                private.as_mut_ptr(),
                lds.as_mut_ptr(),
                CAP,
                &mut count,
            )
        })?;
        Ok((0..count.min(CAP))
            .map(|i| {
                // SAFETY: slot i holds a NUL-terminated name.
                let n = unsafe { CStr::from_ptr(names.as_ptr().add(64 * i)) }.to_string_lossy().into_owned();
                (n, regs[i], private[i], lds[i])
            })
            .collect())
    }
}

impl Drop for HipDevice {
    fn drop(&mut self) {
        // SAFETY: the handle came from hs_device_open; models and batches borrow the device.
        unsafe { ffi::hs_device_close(self.raw) }
    }
}

/// A model file in GPU memory (`hardshell_cuda::CudaModel`).
pub struct HipModel<'d> {
    raw: *mut ffi::hs_model,
    dev: &'d HipDevice,
}

impl std::fmt::Debug for HipModel<'_> {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        f.debug_struct("HipModel").field("hash", &self.hash()).finish_non_exhaustive()
    }
}

impl<'d> HipModel<'d> {
    /// Loads a model file with the accept/reject set of `hardshell::gpt2::Model::load`.
    ///
    /// # Errors
    /// [`Error::Model`] for a file the reference refuses; [`Error::Unsupported`] for head
    /// dims the kernels do not take; [`Error::Hip`] for the upload.
    pub fn load(dev: &'d HipDevice, bytes: &[u8]) -> Result<Self> {
        let mut raw = core::ptr::null_mut();
        // SAFETY: `bytes` is valid for its length; `raw` is a valid out-pointer.
        check("hs_model_load", unsafe { ffi::hs_model_load(dev.raw, bytes.as_ptr(), bytes.len(), &mut raw) })?;
        Ok(Self { raw, dev })
    }

    /// [`HipModel::load`] that reuses the parse of `loaded` when the file is the same
    /// (`CudaModel::load_with`, `model.rs:259-349`). The CPU model of the reference is not
    /// needed: the library keeps its own parse.
    ///
    /// # Errors
    /// As [`HipModel::load`].
    pub fn load_with(dev: &'d HipDevice, bytes: &[u8], loaded: Option<&HipModel<'_>>) -> Result<Self> {
        let mut raw = core::ptr::null_mut();
        let prev = loaded.map_or(core::ptr::null(), |m| m.raw.cast_const());
        // SAFETY: as in load; `prev` is null or a live model.
        check("hs_model_load_with", unsafe {
            ffi::hs_model_load_with(dev.raw, bytes.as_ptr(), bytes.len(), prev, &mut raw)
        })?;
        Ok(Self { raw, dev })
    }

    /// The SHA-256 of the model file.
    #[must_use]
    pub fn hash(&self) -> ModelHash {
        let mut out = [0u8; 32];
        // SAFETY: 32 bytes of output.
        unsafe { ffi::hs_model_hash(self.raw, out.as_mut_ptr()) };
        ModelHash::from_bytes(out)
    }

    /// The vocabulary size.
    #[must_use]
    pub fn vocab_size(&self) -> usize {
        // SAFETY: a getter of a live model.
        unsafe { ffi::hs_model_vocab(self.raw) as usize }
    }

    /// The context length.
    #[must_use]
    pub fn n_ctx(&self) -> usize {
        // SAFETY: a getter of a live model.
        unsafe { ffi::hs_model_n_ctx(self.raw) as usize }
    }

    /// The end-of-text token.
    #[must_use]
    pub fn eot_token(&self) -> TokenId {
        // SAFETY: a getter of a live model.
        TokenId::new(unsafe { ffi::hs_model_eot(self.raw) })
    }

    /// A model of file version 2 (i16 activations).
    #[must_use]
    pub fn is_wide(&self) -> bool {
        // SAFETY: a getter of a live model.
        unsafe { ffi::hs_model_is_wide(self.raw) != 0 }
    }

    /// The device the model is on.
    #[must_use]
    pub fn device(&self) -> &'d HipDevice {
        self.dev
    }

    /// The bytes of the weights on the device.
    #[must_use]
    pub fn weight_bytes(&self) -> u64 {
        // SAFETY: a getter of a live model.
        unsafe { ffi::hs_model_weight_bytes(self.raw) }
    }

    /// The KV-cache bytes of one slot (`2 L n_ctx d`).
    #[must_use]
    pub fn cache_bytes_per_slot(&self) -> u64 {
        // SAFETY: a getter of a live model.
        unsafe { ffi::hs_model_cache_bytes_per_slot(self.raw) }
    }
}

impl Drop for HipModel<'_> {
    fn drop(&mut self) {
        // SAFETY: the handle came from hs_model_load*; batches borrow the model.
        unsafe { ffi::hs_model_free(self.raw) }
    }
}

/// Many independent sessions of one model on one GPU (`hardshell_cuda::CudaBatch`).
pub struct HipBatch<'m> {
    raw: *mut ffi::hs_batch,
    model: &'m HipModel<'m>,
    slots: usize,
    overlap: Overlap,
    weights: Vec<u64>,  // the last step's weights of every slot (`step` / `weights`)
    stepped: Vec<bool>,
}

impl std::fmt::Debug for HipBatch<'_> {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        f.debug_struct("HipBatch").field("slots", &self.slots).finish_non_exhaustive()
    }
}

fn inputs_of(inputs: &[(usize, TokenId)], slots: usize) -> Result<Vec<ffi::hs_input>> {
    inputs
        .iter()
        .map(|&(slot, t)| {
            if slot >= slots {
                return Err(Error::BadSlot { slot, slots });
            }
            let slot = u32::try_from(slot).map_err(|_| Error::BadSlot { slot, slots })?;
            Ok(ffi::hs_input { slot, token: t.get() })
        })
        .collect()
}

fn queries_of(queries: &[CoderQuery]) -> Result<Vec<ffi::hs_query>> {
    queries
        .iter()
        .map(|q| match *q {
            CoderQuery::Encode(t) => Ok(ffi::hs_query { kind: 0, value: t.get() }),
            CoderQuery::Decode(v) => u32::try_from(v)
                .map(|value| ffi::hs_query { kind: 1, value })
                .map_err(|_| Error::Unsupported { reason: "a decode target is not below 2^32".to_owned() }),
        })
        .collect()
}

/// The host mixer behind the C callback. A panic must not cross the FFI boundary: it gives
/// q = 0, which the library refuses (the call fails with Unsupported).
unsafe extern "C" fn trampoline<F: FnMut(usize, MixStats) -> u32>(
    user: *mut c_void,
    input: usize,
    stats: *const ffi::hs_mix_stats,
) -> u32 {
    // SAFETY: `user` is the `&mut F` passed by the caller below for the duration of the call;
    // `stats` points to the library's statistics of this input.
    let (f, s) = unsafe { (&mut *user.cast::<F>(), &*stats) };
    std::panic::catch_unwind(std::panic::AssertUnwindSafe(|| {
        f(input, MixStats { total: s.total, predicted: s.predicted, top: TokenId::new(s.top) })
    }))
    .unwrap_or(0)
}

impl<'m> HipBatch<'m> {
    /// A batch of `slots` slots whose passes hold up to `max_rows` rows (`CudaBatch::new`).
    ///
    /// # Errors
    /// [`Error::Hip`] if the KV caches or work buffers do not fit in device memory.
    pub fn new(model: &'m HipModel<'m>, slots: usize, max_rows: usize) -> Result<Self> {
        let mut raw = core::ptr::null_mut();
        // SAFETY: a live model and a valid out-pointer.
        check("hs_batch_new", unsafe { ffi::hs_batch_new(model.raw, slots, max_rows, &mut raw) })?;
        let vocab = model.vocab_size();
        Ok(Self {
            raw,
            model,
            slots,
            overlap: Overlap::NONE,
            weights: vec![0; slots * vocab],
            stepped: vec![false; slots],
        })
    }

    /// The context overlap (ADR 0015): a full context restarts with EOT and the last `k`
    /// tokens.
    ///
    /// # Errors
    /// [`Error::Model`] if the overlap does not fit the context.
    pub fn set_overlap(&mut self, overlap: Overlap) -> Result<()> {
        // SAFETY: a live batch.
        check("hs_batch_set_overlap", unsafe { ffi::hs_batch_set_overlap(self.raw, u32::from(overlap.get())) })?;
        self.overlap = overlap;
        Ok(())
    }

    /// The context overlap.
    #[must_use]
    pub fn overlap(&self) -> Overlap {
        self.overlap
    }

    /// The number of slots.
    #[must_use]
    pub fn slots(&self) -> usize {
        self.slots
    }

    /// The most rows of one pass.
    #[must_use]
    pub fn max_rows(&self) -> usize {
        // SAFETY: a live batch.
        unsafe { ffi::hs_batch_max_rows(self.raw) }
    }

    /// The device memory of the batch.
    #[must_use]
    pub fn gpu_bytes(&self) -> u64 {
        // SAFETY: a live batch.
        unsafe { ffi::hs_batch_gpu_bytes(self.raw) }
    }

    /// The next position of `slot`.
    #[must_use]
    pub fn position(&self, slot: usize) -> usize {
        // SAFETY: a live batch; the library ignores a slot out of range (0).
        unsafe { ffi::hs_batch_position(self.raw, slot) }
    }

    /// Starts `slot` again at position 0.
    pub fn reset(&mut self, slot: usize) {
        // SAFETY: a live batch; the library ignores a slot out of range.
        unsafe { ffi::hs_batch_reset(self.raw, slot) };
        if let Some(s) = self.stepped.get_mut(slot) {
            *s = false;
        }
    }

    /// The weights of `slot` after the last [`HipBatch::step`] that fed it, if any.
    #[must_use]
    pub fn weights(&self, slot: usize) -> Option<&[u64]> {
        let v = self.model.vocab_size();
        self.stepped.get(slot).copied().unwrap_or(false).then(|| &self.weights[slot * v..(slot + 1) * v])
    }

    /// One token for each of some slots (each slot at most once); their weights are then
    /// [`HipBatch::weights`].
    ///
    /// # Errors
    /// [`Error::BadSlot`], [`Error::Model`] for a token out of range, [`Error::Hip`].
    pub fn step(&mut self, inputs: &[(usize, TokenId)]) -> Result<()> {
        let w = self.run_weights(inputs)?;
        let v = self.model.vocab_size();
        for (i, &(slot, _)) in inputs.iter().enumerate() {
            self.weights[slot * v..(slot + 1) * v].copy_from_slice(&w[i * v..(i + 1) * v]);
            self.stepped[slot] = true;
        }
        Ok(())
    }

    /// The weights of every input, in input order (`inputs.len() * vocab` values). A slot may
    /// occur many times (prefill); its rows run at consecutive positions.
    ///
    /// # Errors
    /// As [`HipBatch::step`]; after an error no position changed.
    pub fn run_weights(&mut self, inputs: &[(usize, TokenId)]) -> Result<Vec<u64>> {
        let ins = inputs_of(inputs, self.slots)?;
        let mut out = vec![0u64; ins.len() * self.model.vocab_size()];
        // SAFETY: `out` holds n * vocab values.
        check("hs_batch_run_weights", unsafe {
            ffi::hs_batch_run_weights(self.raw, ins.as_ptr(), ins.len(), out.as_mut_ptr())
        })?;
        Ok(out)
    }

    /// The passes of `inputs` with nothing read back (`CudaBatch::run_without_readback`).
    ///
    /// # Errors
    /// As [`HipBatch::run_weights`].
    pub fn run_without_readback(&mut self, inputs: &[(usize, TokenId)]) -> Result<()> {
        let ins = inputs_of(inputs, self.slots)?;
        // SAFETY: a live batch and `ins.len()` inputs.
        check("hs_batch_run_without_readback", unsafe {
            ffi::hs_batch_run_without_readback(self.raw, ins.as_ptr(), ins.len())
        })
    }

    /// The coder interval of each input (`CudaBatch::run_coded`): the interval of the query's
    /// token, or the symbol at the query's target, in `FreqTable::from_weights(w, freq_bits)`.
    ///
    /// # Errors
    /// [`Error::LengthMismatch`] if the queries do not match the inputs; as
    /// [`HipBatch::run_weights`] otherwise.
    pub fn run_coded(
        &mut self,
        inputs: &[(usize, TokenId)],
        queries: &[CoderQuery],
        freq_bits: u32,
    ) -> Result<Vec<CoderInterval>> {
        if queries.len() != inputs.len() {
            return Err(Error::LengthMismatch { expected: inputs.len(), found: queries.len() });
        }
        let ins = inputs_of(inputs, self.slots)?;
        let qs = queries_of(queries)?;
        let mut out = vec![ffi::hs_interval::default(); ins.len()];
        // SAFETY: every array holds n entries.
        check("hs_batch_run_coded", unsafe {
            ffi::hs_batch_run_coded(self.raw, ins.as_ptr(), qs.as_ptr(), ins.len(), freq_bits, out.as_mut_ptr())
        })?;
        Ok(self.intervals(&out))
    }

    /// The coder interval of each input in its table (`CudaBatch::run_coded_mixed`): GPT-2
    /// alone or the mixer's weights with the prediction; `mixer` is the host step.
    ///
    /// # Errors
    /// As [`HipBatch::run_coded`]; [`Error::Unsupported`] for a q outside `1..=65535`.
    pub fn run_coded_mixed<F>(
        &mut self,
        inputs: &[(usize, TokenId)],
        queries: &[CoderQuery],
        tables: &[MixInput],
        freq_bits: u32,
        mut mixer: F,
    ) -> Result<Vec<CoderInterval>>
    where
        F: FnMut(usize, MixStats) -> u32,
    {
        if queries.len() != inputs.len() || tables.len() != inputs.len() {
            let found = if queries.len() != inputs.len() { queries.len() } else { tables.len() };
            return Err(Error::LengthMismatch { expected: inputs.len(), found });
        }
        let ins = inputs_of(inputs, self.slots)?;
        let qs = queries_of(queries)?;
        let ts: Vec<u32> = tables
            .iter()
            .map(|t| match *t {
                MixInput::Plain => HS_MIX_PLAIN,
                MixInput::Mixed(None) => HS_MIX_NONE,
                MixInput::Mixed(Some(p)) => p.get(),
            })
            .collect();
        let mut out = vec![ffi::hs_interval::default(); ins.len()];
        // SAFETY: every array holds n entries; `mixer` outlives the call.
        check("hs_batch_run_coded_mixed", unsafe {
            ffi::hs_batch_run_coded_mixed(
                self.raw,
                ins.as_ptr(),
                qs.as_ptr(),
                ts.as_ptr(),
                ins.len(),
                freq_bits,
                Some(trampoline::<F>),
                (&mut mixer as *mut F).cast(),
                out.as_mut_ptr(),
            )
        })?;
        Ok(self.intervals(&out))
    }

    /// For each input the interval of `tokens[i]` in the table of GPT-2 alone and in the mixed
    /// table with `predictions[i]`, from one pass (`CudaBatch::run_coded_dual`).
    ///
    /// # Errors
    /// As [`HipBatch::run_coded_mixed`].
    pub fn run_coded_dual<F>(
        &mut self,
        inputs: &[(usize, TokenId)],
        tokens: &[TokenId],
        predictions: &[Option<TokenId>],
        freq_bits: u32,
        mut mixer: F,
    ) -> Result<Vec<(CoderInterval, CoderInterval)>>
    where
        F: FnMut(usize, MixStats) -> u32,
    {
        if tokens.len() != inputs.len() || predictions.len() != inputs.len() {
            let found = if tokens.len() != inputs.len() { tokens.len() } else { predictions.len() };
            return Err(Error::LengthMismatch { expected: inputs.len(), found });
        }
        let ins = inputs_of(inputs, self.slots)?;
        let toks: Vec<u32> = tokens.iter().map(|t| t.get()).collect();
        let preds: Vec<u32> = predictions.iter().map(|p| p.map_or(HS_MIX_NONE, TokenId::get)).collect();
        let mut plain = vec![ffi::hs_interval::default(); ins.len()];
        let mut mixed = vec![ffi::hs_interval::default(); ins.len()];
        // SAFETY: every array holds n entries; `mixer` outlives the call.
        check("hs_batch_run_coded_dual", unsafe {
            ffi::hs_batch_run_coded_dual(
                self.raw,
                ins.as_ptr(),
                toks.as_ptr(),
                preds.as_ptr(),
                ins.len(),
                freq_bits,
                Some(trampoline::<F>),
                (&mut mixer as *mut F).cast(),
                plain.as_mut_ptr(),
                mixed.as_mut_ptr(),
            )
        })?;
        Ok(self.intervals(&plain).into_iter().zip(self.intervals(&mixed)).collect())
    }

    /// The inputs of `slot` since its last reset (`batch/stream.rs:19-24`).
    #[must_use]
    pub fn stream_len(&self, slot: usize) -> usize {
        // SAFETY: a live batch.
        unsafe { ffi::hs_batch_stream_len(self.raw, slot) }
    }

    /// The inputs `slot` takes before its next restart (`batch/stream.rs:27-34`).
    #[must_use]
    pub fn room(&self, slot: usize) -> usize {
        // SAFETY: a live batch.
        unsafe { ffi::hs_batch_room(self.raw, slot) }
    }

    /// Cuts the stream of `slot` back to `len` inputs (speculative drafts,
    /// `batch/stream.rs:46-75`).
    ///
    /// # Errors
    /// [`Error::BadSlot`]; [`Error::Model`] for a truncation the stream rules refuse.
    pub fn truncate(&mut self, slot: usize, len: usize) -> Result<()> {
        if slot >= self.slots {
            return Err(Error::BadSlot { slot, slots: self.slots });
        }
        // SAFETY: a live batch and a slot in range.
        check("hs_batch_truncate", unsafe { ffi::hs_batch_truncate(self.raw, slot, len) })?;
        self.stepped[slot] = false;
        Ok(())
    }

    fn intervals(&self, out: &[ffi::hs_interval]) -> Vec<CoderInterval> {
        let vocab = self.model.vocab_size() as u64;
        out.iter()
            .map(|i| CoderInterval {
                symbol: TokenId::new(i.symbol as u32),
                start: i.start,
                freq: i.freq,
                is_last: i.symbol + 1 == vocab,
            })
            .collect()
    }
}

impl Drop for HipBatch<'_> {
    fn drop(&mut self) {
        // SAFETY: the handle came from hs_batch_new.
        unsafe { ffi::hs_batch_free(self.raw) }
    }
}

/// One session: a batch of one slot with the API shape of `hardshell::gpt2::Session`
/// (`hardshell_cuda::CudaSession`).
#[derive(Debug)]
pub struct HipSession<'m> {
    batch: HipBatch<'m>,
}

impl<'m> HipSession<'m> {
    /// A session with no context overlap.
    ///
    /// # Errors
    /// As [`HipBatch::new`].
    pub fn new(model: &'m HipModel<'m>) -> Result<Self> {
        Self::with_overlap(model, Overlap::NONE)
    }

    /// A session with the context overlap `overlap`.
    ///
    /// # Errors
    /// As [`HipBatch::new`] and [`HipBatch::set_overlap`].
    pub fn with_overlap(model: &'m HipModel<'m>, overlap: Overlap) -> Result<Self> {
        let mut batch = HipBatch::new(model, 1, 64)?;
        batch.set_overlap(overlap)?;
        Ok(Self { batch })
    }

    /// Starts again at position 0.
    pub fn reset(&mut self) {
        self.batch.reset(0);
    }

    /// The next position.
    #[must_use]
    pub fn position(&self) -> usize {
        self.batch.position(0)
    }

    /// The weights of the first token of a block: the step of EOT at position 0.
    ///
    /// # Errors
    /// As [`HipSession::step`].
    pub fn start_block(&mut self) -> Result<&[u64]> {
        self.reset();
        let eot = self.batch.model.eot_token();
        self.step(eot)
    }

    /// The inputs since the last reset.
    #[must_use]
    pub fn stream_len(&self) -> usize {
        self.batch.stream_len(0)
    }

    /// Cuts the stream back to `len` inputs.
    ///
    /// # Errors
    /// As [`HipBatch::truncate`].
    pub fn truncate(&mut self, len: usize) -> Result<()> {
        self.batch.truncate(0, len)
    }

    /// One token; the weights of the next one.
    ///
    /// # Errors
    /// As [`HipBatch::step`].
    pub fn step(&mut self, token: TokenId) -> Result<&[u64]> {
        self.batch.step(&[(0, token)])?;
        self.batch.weights(0).ok_or(Error::Unsupported { reason: "no weights after a step".to_owned() })
    }
}

/// The library's version string, with the SHA-256 prefix of the kernel sources it was built
/// from.
#[must_use]
pub fn version() -> String {
    // SAFETY: a static NUL-terminated string.
    unsafe { CStr::from_ptr(ffi::hs_version()) }.to_string_lossy().into_owned()
}
