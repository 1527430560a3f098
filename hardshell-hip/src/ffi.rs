//! The C ABI of `libhardshell_hip.so`, one declaration for each function of
//! `include/hardshell_hip.h` (the header is the contract; its comments cite the reference
//! interface each entry replaces). Every pointer is a plain host or device pointer; the
//! handles are opaque. Every `hs_status` is a `c_int` with the values of [`Status`].

#![allow(non_camel_case_types)]

use core::ffi::{c_char, c_int, c_void};

/// `hs_device`: one GPU with the kernels loaded (`CudaDevice`).
#[repr(C)]
pub struct hs_device {
    _opaque: [u8; 0],
}

/// `hs_model`: a model file in GPU memory (`CudaModel`).
#[repr(C)]
pub struct hs_model {
    _opaque: [u8; 0],
}

/// `hs_batch`: the slots of one model (`CudaBatch`).
#[repr(C)]
pub struct hs_batch {
    _opaque: [u8; 0],
}

/// One `(slot, token)` input.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct hs_input {
    pub slot: u32,
    pub token: u32,
}

/// A coder query: `kind` 0 is Encode(token = value), 1 is Decode(target = value).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct hs_query {
    pub kind: u32,
    pub value: u32,
}

/// The interval of one symbol; the last symbol is `symbol + 1 == vocab`.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct hs_interval {
    pub symbol: u64,
    pub start: u64,
    pub freq: u64,
}

/// The statistics of one input's weights for the host mixer.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct hs_mix_stats {
    pub total: u64,
    pub predicted: u64,
    pub top: u32,
    pub pad: u32,
}

/// The host step of the mixed coder op: `q` in `1..=65535` for input `input`.
pub type hs_mixer_fn = Option<unsafe extern "C" fn(user: *mut c_void, input: usize, stats: *const hs_mix_stats) -> u32>;

/// A mixed table without a prediction.
pub const HS_MIX_NONE: u32 = 0xFFFF_FFFF;
/// The table of GPT-2 alone.
pub const HS_MIX_PLAIN: u32 = 0xFFFF_FFFE;

/// The values of `hs_status`.
#[repr(i32)]
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Status {
    Ok = 0,
    NoDevice = 1,
    DeviceError = 2,
    Unsupported = 3,
    ModelError = 4,
    BadSlot = 5,
    LengthMismatch = 6,
    InvalidArgument = 7,
}

#[link(name = "hardshell_hip")]
unsafe extern "C" {
    // ---- errors and version
    pub fn hs_last_error_message() -> *const c_char;
    pub fn hs_last_error_code() -> c_int;
    pub fn hs_version() -> *const c_char;

    // ---- device
    pub fn hs_device_open(ordinal: c_int, out: *mut *mut hs_device) -> c_int;
    pub fn hs_device_close(dev: *mut hs_device);
    pub fn hs_device_name(dev: *const hs_device, buf: *mut c_char, cap: usize) -> c_int;
    pub fn hs_device_memory(dev: *const hs_device, free_bytes: *mut usize, total_bytes: *mut usize) -> c_int;
    pub fn hs_device_kernel_resources(
        dev: *mut hs_device,
        names: *mut c_char,
        regs: *mut i32,
        private_bytes: *mut i32,
        static_lds: *mut i32,
        cap: usize,
        count: *mut usize,
    ) -> c_int;

    // ---- model
    pub fn hs_model_load(dev: *mut hs_device, bytes: *const u8, len: usize, out: *mut *mut hs_model) -> c_int;
    pub fn hs_model_load_with(
        dev: *mut hs_device,
        bytes: *const u8,
        len: usize,
        loaded: *const hs_model,
        out: *mut *mut hs_model,
    ) -> c_int;
    pub fn hs_model_free(model: *mut hs_model);
    pub fn hs_model_validate(bytes: *const u8, len: usize, hash: *mut u8) -> c_int;
    pub fn hs_model_hash(model: *const hs_model, out: *mut u8);
    pub fn hs_model_vocab(model: *const hs_model) -> u32;
    pub fn hs_model_n_ctx(model: *const hs_model) -> u32;
    pub fn hs_model_eot(model: *const hs_model) -> u32;
    pub fn hs_model_is_wide(model: *const hs_model) -> c_int;
    pub fn hs_model_token(model: *const hs_model, id: u32, bytes: *mut *const u8, len: *mut usize) -> c_int;
    pub fn hs_model_merges(model: *const hs_model, pairs: *mut *const u32) -> usize;
    pub fn hs_model_weight_bytes(model: *const hs_model) -> u64;
    pub fn hs_model_cache_bytes_per_slot(model: *const hs_model) -> u64;

    // ---- batch
    pub fn hs_batch_new(model: *mut hs_model, slots: usize, max_rows: usize, out: *mut *mut hs_batch) -> c_int;
    pub fn hs_batch_free(batch: *mut hs_batch);
    pub fn hs_batch_set_overlap(batch: *mut hs_batch, k: u32) -> c_int;
    pub fn hs_batch_slots(batch: *const hs_batch) -> usize;
    pub fn hs_batch_model(batch: *const hs_batch) -> *const hs_model;
    pub fn hs_batch_max_rows(batch: *const hs_batch) -> usize;
    pub fn hs_batch_gpu_bytes(batch: *const hs_batch) -> u64;
    pub fn hs_batch_position(batch: *const hs_batch, slot: usize) -> usize;
    pub fn hs_batch_reset(batch: *mut hs_batch, slot: usize);
    pub fn hs_batch_run_weights(batch: *mut hs_batch, inputs: *const hs_input, n: usize, out: *mut u64) -> c_int;
    pub fn hs_batch_run_without_readback(batch: *mut hs_batch, inputs: *const hs_input, n: usize) -> c_int;
    pub fn hs_batch_run_coded(
        batch: *mut hs_batch,
        inputs: *const hs_input,
        queries: *const hs_query,
        n: usize,
        freq_bits: u32,
        out: *mut hs_interval,
    ) -> c_int;
    pub fn hs_batch_step(batch: *mut hs_batch, inputs: *const hs_input, n: usize) -> c_int;
    pub fn hs_batch_weights(batch: *const hs_batch, slot: usize, out: *mut u64) -> c_int;
    pub fn hs_batch_stream_len(batch: *const hs_batch, slot: usize) -> usize;
    pub fn hs_batch_room(batch: *const hs_batch, slot: usize) -> usize;
    pub fn hs_batch_truncate(batch: *mut hs_batch, slot: usize, len: usize) -> c_int;
    pub fn hs_batch_run_coded_mixed(
        batch: *mut hs_batch,
        inputs: *const hs_input,
        queries: *const hs_query,
        tables: *const u32,
        n: usize,
        freq_bits: u32,
        mixer: hs_mixer_fn,
        user: *mut c_void,
        out: *mut hs_interval,
    ) -> c_int;
    pub fn hs_batch_run_coded_dual(
        batch: *mut hs_batch,
        inputs: *const hs_input,
        tokens: *const u32,
        predictions: *const u32,
        n: usize,
        freq_bits: u32,
        mixer: hs_mixer_fn,
        user: *mut c_void,
        plain: *mut hs_interval,
        mixed: *mut hs_interval,
    ) -> c_int;

    // ---- op-level entries (tests and measurements)
    pub fn hs_op_mixed_coder(
        dev: *mut hs_device,
        weights: *const u64,
        rows: usize,
        vocab: usize,
        queries: *const hs_query,
        predictions: *const u32,
        freq_bits: u32,
        mixer: hs_mixer_fn,
        user: *mut c_void,
        stats: *mut hs_mix_stats,
        out: *mut hs_interval,
    ) -> c_int;
    pub fn hs_op_mixed_coder_logits(
        dev: *mut hs_device,
        logits: *const i64,
        rows: usize,
        vocab: usize,
        table: *const u64,
        len: usize,
        queries: *const hs_query,
        tables: *const u32,
        freq_bits: u32,
        mixer: hs_mixer_fn,
        user: *mut c_void,
        stats: *mut hs_mix_stats,
        out: *mut hs_interval,
    ) -> c_int;
    pub fn hs_op_gemm_i8(dev: *mut hs_device, w: *const i8, a: *const i8, m: usize, n: usize, k: usize, out: *mut i32) -> c_int;
    pub fn hs_op_gemm_i8_split(
        dev: *mut hs_device,
        w: *const i8,
        a: *const i8,
        m: usize,
        n: usize,
        k: usize,
        splits: u32,
        out: *mut i32,
    ) -> c_int;
    pub fn hs_op_gemm_i8_i16(
        dev: *mut hs_device,
        w: *const i8,
        a: *const i16,
        m: usize,
        n: usize,
        k: usize,
        splits: u32,
        out: *mut i64,
    ) -> c_int;
    pub fn hs_op_gemm_requant_i8(
        dev: *mut hs_device,
        w: *const i8,
        a: *const i8,
        bias: *const i32,
        mult: *const i32,
        shift: u8,
        m: usize,
        n: usize,
        k: usize,
        out: *mut i8,
    ) -> c_int;
    pub fn hs_op_gemm_requant_i8_dev(
        dev: *mut hs_device,
        w: *const i8,
        a: *const i8,
        bias: *const i32,
        mult: *const i32,
        shift: u8,
        m: usize,
        n: usize,
        k: usize,
        out: *mut i8,
        stream: *mut c_void,
    ) -> c_int;
    pub fn hs_op_gemm_layout(m: usize, n: usize, k: usize, m_pad: *mut usize, n_pad: *mut usize, k_pad: *mut usize);
    pub fn hs_op_attend_decode_dev(
        dev: *mut hs_device,
        q: *const i8,
        k_cache: *const i8,
        v_cache: *const i8,
        ctx: *const u32,
        b: usize,
        h: usize,
        hd: usize,
        ctx_cap: usize,
        score_m: i32,
        score_s: u8,
        out_m: i32,
        out_s: u8,
        attn_exp: *const i32,
        len: usize,
        softmax_p: u8,
        out: *mut i8,
        stream: *mut c_void,
    ) -> c_int;
    /// No counterpart in the reference: decode attention with no allocation (for callers that
    /// cannot allocate, such as code under HIP graph capture).
    pub fn hs_op_attend_decode_dev_noalloc(
        dev: *mut hs_device,
        q: *const i8,
        k_cache: *const i8,
        v_cache: *const i8,
        ctx: *const u32,
        b: usize,
        h: usize,
        hd: usize,
        ctx_cap: usize,
        score_m: i32,
        score_s: u8,
        out_m: i32,
        out_s: u8,
        attn_exp: *const i32,
        len: usize,
        softmax_p: u8,
        out: *mut i8,
        stream: *mut c_void,
    ) -> c_int;
    pub fn hs_op_coder(
        dev: *mut hs_device,
        logits: *const i64,
        rows: usize,
        vocab: usize,
        table: *const u64,
        len: usize,
        queries: *const hs_query,
        freq_bits: u32,
        out: *mut hs_interval,
    ) -> c_int;
    pub fn hs_op_gemm_requant_gpu_ns(
        dev: *mut hs_device,
        w: *const i8,
        a: *const i8,
        bias: *const i32,
        mult: *const i32,
        shift: u8,
        m: usize,
        n: usize,
        k: usize,
        out: *mut i8,
        reps: usize,
        ns: *mut u64,
    ) -> c_int;
    pub fn hs_op_attend_decode_gpu_ns(
        dev: *mut hs_device,
        q: *const i8,
        k_cache: *const i8,
        v_cache: *const i8,
        ctx: *const u32,
        b: usize,
        h: usize,
        hd: usize,
        ctx_cap: usize,
        score_m: i32,
        score_s: u8,
        out_m: i32,
        out_s: u8,
        attn_exp: *const i32,
        len: usize,
        softmax_p: u8,
        out: *mut i8,
        reps: usize,
        ns: *mut u64,
    ) -> c_int;
    /// No counterpart in the reference: one timed launch on each of `sets` cache sets in turn.
    pub fn hs_op_attend_decode_sets_gpu_ns(
        dev: *mut hs_device,
        q: *const i8,
        k_caches: *const *const i8,
        v_caches: *const *const i8,
        sets: usize,
        ctx: *const u32,
        b: usize,
        h: usize,
        hd: usize,
        ctx_cap: usize,
        score_m: i32,
        score_s: u8,
        out_m: i32,
        out_s: u8,
        attn_exp: *const i32,
        len: usize,
        softmax_p: u8,
        out: *mut i8,
        ns: *mut u64,
    ) -> c_int;
    pub fn hs_read_bw(dev: *mut hs_device, bytes: usize, reps: usize, ns: *mut u64) -> c_int;
    /// No counterpart in the reference: the VALU / MFMA issue-rate probe.
    pub fn hs_probe_issue(dev: *mut hs_device, op: u32, waves_per_simd: u32, iters: u32, ns: *mut u64) -> c_int;

    // ---- profiling
    pub fn hs_batch_set_profiling(batch: *mut hs_batch, on: c_int) -> c_int;
    pub fn hs_batch_profile(
        batch: *mut hs_batch,
        labels: *mut c_char,
        ns: *mut u64,
        launches: *mut u64,
        ops: *mut u64,
        cap: usize,
        clear: c_int,
    ) -> usize;

    // ---- device memory (test and measurement plumbing)
    pub fn hs_device_alloc(dev: *mut hs_device, bytes: usize, out: *mut *mut c_void) -> c_int;
    pub fn hs_device_free(dev: *mut hs_device, ptr: *mut c_void);
    pub fn hs_device_upload(dev: *mut hs_device, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn hs_device_download(dev: *mut hs_device, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn hs_device_synchronize(dev: *mut hs_device) -> c_int;
    pub fn hs_device_copy(dev: *mut hs_device, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
}
