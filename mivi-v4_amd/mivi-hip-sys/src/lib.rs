//! Rust binding of `libmivi_hip.so`, the MI355X (gfx950) implementation of
//! mivi-v4's quantized-inference hot path (`include/mivi_hip.h`).
//!
//! * `ffi`: the C ABI one-to-one, every function of the header.
//! * `quant`: `GgmlType` and `QuantError` as `crates/mivi-quant/src/types.rs`
//!   defines them, and safe wrappers with the signatures of
//!   `mivi_quant::quantized_matvec` (`lib.rs:75-82`),
//!   `quantized_matmul_rows` (`lib.rs:136-151`) and `dequantize_slice`
//!   (`lib.rs:35`) over host slices, which stage the buffers through device
//!   memory; and the same calls over device buffers (`DeviceBuffer`), which is
//!   how a decode loop keeps weights resident.
//!
//! The image this crate was written in has no Rust toolchain: it has not been
//! compiled. `tests/test_ffi_crate.py` checks the extern block against the
//! header, symbol for symbol and argument for argument.

#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_void};

pub mod ffi {
    use super::*;

    #[repr(C)]
    pub struct MiviError {
        pub code: i32,
        pub type_id: u32,
        pub expected: usize,
        pub actual: usize,
        pub dim: usize,
        pub block_size: usize,
        pub message: [c_char; 256],
    }

    #[repr(C)]
    pub struct MiviModel {
        _private: [u8; 0],
    }

    #[repr(C)]
    pub struct MiviPrefixCache {
        _private: [u8; 0],
    }

    /// GenerationConfig's sampling fields (config.rs:163-174); top_k 0 = off.
    #[repr(C)]
    #[derive(Clone, Copy, Debug)]
    pub struct MiviSamplerConfig {
        pub temperature: f32,
        pub top_p: f32,
        pub min_p: f32,
        pub repetition_penalty: f32,
        pub presence_penalty: f32,
        pub frequency_penalty: f32,
        pub top_k: u32,
    }

    #[repr(C)]
    #[derive(Default, Debug, Clone, Copy)]
    pub struct MiviModelInfo {
        pub dim: usize,
        pub hidden_dim: usize,
        pub n_layers: usize,
        pub n_heads: usize,
        pub n_kv_heads: usize,
        pub head_dim: usize,
        pub kv_dim: usize,
        pub vocab_size: usize,
        pub max_seq_len: usize,
        pub ssm_conv_kernel: usize,
        pub n_attn_layers: usize,
        pub max_batch: usize,
        pub rope_base: f32,
        pub rms_norm_eps: f32,
        pub kv_precision: i32,
        pub yarn: i32,
        pub yarn_scale: f32,
        pub weight_bytes: usize,
        pub kv_bytes: usize,
    }

    pub const MIVI_OK: i32 = 0;
    pub const MIVI_ERR_UNSUPPORTED_TYPE: i32 = 1;
    pub const MIVI_ERR_BUFFER_TOO_SMALL: i32 = 2;
    pub const MIVI_ERR_DIMENSION_MISALIGNED: i32 = 3;
    pub const MIVI_ERR_ARITHMETIC_OVERFLOW: i32 = 4;
    pub const MIVI_ERR_HIP: i32 = 100;
    pub const MIVI_ERR_INVALID_ARGUMENT: i32 = 101;
    pub const MIVI_ERR_INVALID_TOKEN: i32 = 110;
    pub const MIVI_ERR_CONTEXT_OVERFLOW: i32 = 111;
    pub const MIVI_ERR_GGUF: i32 = 112;
    pub const MIVI_ERR_MISSING_WEIGHT: i32 = 113;
    pub const MIVI_ERR_INVALID_CONFIG: i32 = 114;
    pub const MIVI_ERR_KV_CACHE: i32 = 115;
    pub const MIVI_ERR_UNSUPPORTED: i32 = 116;

    pub const MIVI_KV_F32: i32 = 0;
    pub const MIVI_KV_Q8_0: i32 = 1;
    pub const MIVI_KV_F16: i32 = 2;

    extern "C" {
        pub fn mivi_hip_last_error(out: *mut MiviError) -> i32;
        pub fn mivi_hip_version() -> *const c_char;

        // crates/mivi-quant/src/lib.rs:75-134
        pub fn mivi_hip_quantized_matvec(out: *mut f32, out_len: usize, ggml_type: i32, weights: *const u8,
            weights_len: usize, x: *const f32, x_len: usize, n: usize, d: usize, stream: *mut c_void) -> i32;
        // q4_k_m.rs:217, q6_k.rs:202, q8_0.rs:127, f16.rs:42 / :75
        pub fn mivi_hip_try_matvec_q4_k_m(out: *mut f32, out_len: usize, weights: *const u8, weights_len: usize,
            x: *const f32, x_len: usize, n: usize, d: usize, stream: *mut c_void) -> i32;
        pub fn mivi_hip_try_matvec_q6_k(out: *mut f32, out_len: usize, weights: *const u8, weights_len: usize,
            x: *const f32, x_len: usize, n: usize, d: usize, stream: *mut c_void) -> i32;
        pub fn mivi_hip_try_matvec_q8_0(out: *mut f32, out_len: usize, weights: *const u8, weights_len: usize,
            x: *const f32, x_len: usize, n: usize, d: usize, stream: *mut c_void) -> i32;
        pub fn mivi_hip_try_matvec_f16(out: *mut f32, out_len: usize, weights: *const u8, weights_len: usize,
            x: *const f32, x_len: usize, n: usize, d: usize, stream: *mut c_void) -> i32;
        pub fn mivi_hip_try_matvec_bf16(out: *mut f32, out_len: usize, weights: *const u8, weights_len: usize,
            x: *const f32, x_len: usize, n: usize, d: usize, stream: *mut c_void) -> i32;
        // lib.rs:143-251
        pub fn mivi_hip_quantized_matmul_rows(out: *mut f32, out_len: usize, ggml_type: i32, weights: *const u8,
            weights_len: usize, inputs: *const f32, inputs_len: usize, batch: usize, rows: usize, cols: usize,
            stream: *mut c_void) -> i32;
        // no counterpart in the reference: Q6_K rows repacked once (same
        // size) and the matvec over them, bit-identical to the GGUF-row one
        pub fn mivi_hip_pack_weights(ggml_type: i32, src: *const u8, src_len: usize, dst: *mut u8, dst_len: usize,
            rows: usize, cols: usize, stream: *mut c_void) -> i32;
        pub fn mivi_hip_quantized_matvec_packed(out: *mut f32, out_len: usize, ggml_type: i32, packed: *const u8,
            packed_len: usize, x: *const f32, x_len: usize, n: usize, d: usize, stream: *mut c_void) -> i32;
        pub fn mivi_hip_quantized_matmul_rows_packed(out: *mut f32, out_len: usize, ggml_type: i32,
            packed: *const u8, packed_len: usize, inputs: *const f32, inputs_len: usize, batch: usize, rows: usize,
            cols: usize, stream: *mut c_void) -> i32;
        // the row products' operand layout (no counterpart in the reference)
        pub fn mivi_hip_gemm_packed_size(ggml_type: i32, rows: usize, cols: usize) -> usize;
        pub fn mivi_hip_pack_weights_gemm(ggml_type: i32, src: *const u8, src_len: usize, dst: *mut u8,
            dst_len: usize, rows: usize, cols: usize, stream: *mut c_void) -> i32;
        pub fn mivi_hip_quantized_matmul_rows_gemm_packed(out: *mut f32, out_len: usize, ggml_type: i32,
            weights: *const u8, weights_len: usize, wg: *const u8, wg_len: usize, inputs: *const f32,
            inputs_len: usize, batch: usize, rows: usize, cols: usize, stream: *mut c_void) -> i32;
        // lib.rs:35-72
        pub fn mivi_hip_dequantize_slice(ggml_type: i32, bytes: *const u8, bytes_len: usize, out: *mut f32,
            out_len: usize, stream: *mut c_void) -> i32;
        // q8_0.rs:31-124
        pub fn mivi_hip_quantize_q8_0(src: *const f32, src_len: usize, dst: *mut u8, dst_len: usize,
            n_blocks: usize, stream: *mut c_void) -> i32;
        pub fn mivi_hip_dot_q8_0_f32(q: *const f32, q_len: usize, k_blocks: *const u8, k_len: usize,
            out: *mut f32, out_len: usize, n: usize, stream: *mut c_void) -> i32;

        // crates/mivi-model/src/model.rs:105-606
        pub fn mivi_hip_model_create(gguf: *const u8, gguf_len: usize, max_ctx: usize, kv_precision: i32,
            max_batch: usize, out: *mut *mut MiviModel) -> i32;
        pub fn mivi_hip_model_destroy(m: *mut MiviModel);
        pub fn mivi_hip_model_info(m: *const MiviModel, out: *mut MiviModelInfo) -> i32;
        pub fn mivi_hip_model_reset(m: *mut MiviModel) -> i32;
        pub fn mivi_hip_model_forward_step(m: *mut MiviModel, seq: usize, token: u32, pos: usize,
            compute_logits: i32, logits_host: *mut f32) -> i32;
        pub fn mivi_hip_model_forward(m: *mut MiviModel, seq: usize, token: u32, pos: usize,
            logits_host: *mut f32) -> i32;
        pub fn mivi_hip_model_forward_batch(m: *mut MiviModel, batch: usize, tokens: *const u32, pos: *const usize,
            logits_host: *mut f32) -> i32;
        pub fn mivi_hip_model_generate_greedy(m: *mut MiviModel, batch: usize, tokens: *const u32,
            pos: *const usize, n_steps: usize, tokens_out: *mut u32) -> i32;
        pub fn mivi_hip_model_prefill(m: *mut MiviModel, seq: usize, tokens: *const u32, n: usize,
            pos0: usize) -> i32;
        // Model::set_prefill_strategy (model.rs:260-266): 0/1 = Token, t > 1 = Chunked { tile_tokens: t }
        pub fn mivi_hip_model_set_prefill_tile(m: *mut MiviModel, tile_tokens: usize) -> i32;
        // cache.rs:682-914, arena.rs:110-123
        pub fn mivi_hip_model_export_state(m: *mut MiviModel, seq: usize, tokens: usize, k_out: *mut c_void,
            v_out: *mut c_void, kv_len: usize, conv_out: *mut f32, conv_len: usize) -> i32;
        pub fn mivi_hip_model_import_state(m: *mut MiviModel, seq: usize, tokens: usize, k_in: *const c_void,
            v_in: *const c_void, kv_len: usize, conv_in: *const f32, conv_len: usize) -> i32;
        pub fn mivi_hip_model_export_state_range(m: *mut MiviModel, seq: usize, start: usize, tokens: usize,
            k_out: *mut c_void, v_out: *mut c_void, kv_len: usize, conv_out: *mut f32, conv_len: usize) -> i32;
        pub fn mivi_hip_model_import_state_at(m: *mut MiviModel, seq: usize, start: usize, tokens: usize,
            k_in: *const c_void, v_in: *const c_void, kv_len: usize, conv_in: *const f32, conv_len: usize) -> i32;

        // sampler.rs:91-135 Sampler::sample on the device
        pub fn mivi_hip_sample(logits: *mut f32, n: usize, recent: *const u32, n_recent: usize,
            cfg: *const MiviSamplerConfig, rng_state: *mut u64, token: *mut u32, stream: *mut c_void) -> i32;
        // no counterpart in the reference: mivi_hip_sample with the library's
        // fixed device scratch (n <= 262144), for callers that cannot
        // allocate (graph capture); calls overlapping on one GPU race
        pub fn mivi_hip_sample_noalloc(logits: *mut f32, n: usize, recent: *const u32, n_recent: usize,
            cfg: *const MiviSamplerConfig, rng_state: *mut u64, token: *mut u32, stream: *mut c_void) -> i32;
        pub fn mivi_hip_sample_rows_workspace(n: usize, rows: usize) -> usize;
        pub fn mivi_hip_sample_rows(logits: *mut f32, n: usize, rows: usize, row_stride: usize,
            recent: *const u32, n_recent: usize, recent_stride: usize, cfg: *const MiviSamplerConfig,
            rng_states: *mut u64, tokens: *mut u32, workspace: *mut c_void, workspace_bytes: usize,
            stream: *mut c_void) -> i32;
        // model.rs:1130-1180: the generation loop with the device sampler
        pub fn mivi_hip_model_generate(m: *mut MiviModel, batch: usize, tokens: *const u32, pos: *const usize,
            n_steps: usize, cfg: *const MiviSamplerConfig, seeds: *const u64, eos_ids: *const u32, n_eos: usize,
            tokens_out: *mut u32) -> i32;

        // crates/mivi-kv/src/prefix.rs: PrefixCache with device-resident snapshots
        pub fn mivi_hip_prefix_cache_create(max_chunks: usize, chunk_size: usize, max_memory_bytes: usize,
            out: *mut *mut MiviPrefixCache) -> i32;
        pub fn mivi_hip_prefix_cache_destroy(pc: *mut MiviPrefixCache);
        pub fn mivi_hip_prefix_chunk_hash(prev_hash: u64, tokens: *const u32, n: usize) -> u64;
        pub fn mivi_hip_prefix_cache_insert_delta(pc: *mut MiviPrefixCache, m: *mut MiviModel, seq: usize,
            pos: usize, prev_hash: u64, tokens: *const u32, n_tokens: usize, chunk_index: usize,
            hash_out: *mut u64) -> i32;
        pub fn mivi_hip_prefix_cache_insert(pc: *mut MiviPrefixCache, m: *mut MiviModel, seq: usize, pos: usize,
            prev_hash: u64, tokens: *const u32, n_tokens: usize, chunk_index: usize, hash_out: *mut u64) -> i32;
        pub fn mivi_hip_prefix_cache_find_suffix(pc: *mut MiviPrefixCache, start_pos: usize, tokens: *const u32,
            n: usize, suffix_len: *mut usize, match_pos: *mut usize, hash_out: *mut u64) -> i32;
        pub fn mivi_hip_prefix_cache_find(pc: *mut MiviPrefixCache, tokens: *const u32, n: usize,
            matched: *mut usize, hash_out: *mut u64) -> i32;
        pub fn mivi_hip_prefix_cache_restore(pc: *mut MiviPrefixCache, m: *mut MiviModel, seq: usize,
            tokens: *const u32, n: usize, matched: *mut usize, hash_out: *mut u64) -> i32;
        pub fn mivi_hip_prefix_cache_len(pc: *const MiviPrefixCache) -> usize;
        pub fn mivi_hip_prefix_cache_memory_bytes(pc: *const MiviPrefixCache) -> usize;
        pub fn mivi_hip_prefix_cache_prune(pc: *mut MiviPrefixCache, target_bytes: usize) -> usize;
        pub fn mivi_hip_prefix_cache_clear(pc: *mut MiviPrefixCache);
        pub fn mivi_hip_prefix_cache_contains(pc: *const MiviPrefixCache, hash: u64) -> i32;

        // measurement, no counterpart in the reference
        pub fn mivi_hip_read_floor(p: *const u8, bytes: usize, stream: *mut c_void) -> i32;

        // seeded synthetic inputs (host), no counterpart in the reference
        pub fn mivi_synth_normal(seed: u64, mean: f32, std: f32, out: *mut f32, n: usize);
        pub fn mivi_synth_quantize(ggml_type: i32, src: *const f32, rows: usize, cols: usize, dst: *mut u8,
            dst_len: usize) -> i32;
        pub fn mivi_synth_random_weights(ggml_type: i32, seed: u64, std: f32, rows: usize, cols: usize,
            dst: *mut u8, dst_len: usize) -> i32;
    }

    // The HIP runtime calls the host-slice wrappers below stage through.
    pub const HIP_MEMCPY_HOST_TO_DEVICE: i32 = 1;
    pub const HIP_MEMCPY_DEVICE_TO_HOST: i32 = 2;

    extern "C" {
        pub fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> i32;
        pub fn hipFree(ptr: *mut c_void) -> i32;
        pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, size: usize, kind: i32) -> i32;
        pub fn hipDeviceSynchronize() -> i32;
    }
}

pub mod quant {
    //! `GgmlType`, `QuantError` (crates/mivi-quant/src/types.rs:5-52) and the
    //! `mivi_quant` entry points on the GPU.
    use super::ffi;
    use std::os::raw::c_void;

    /// types.rs:22-52 (the ids this library runs).
    #[derive(Clone, Copy, Debug, PartialEq, Eq)]
    #[repr(u32)]
    pub enum GgmlType {
        F32 = 0,
        F16 = 1,
        Q8_0 = 8,
        Q4_K = 12,
        Q6_K = 14,
        BF16 = 30,
    }

    impl GgmlType {
        pub fn block_size(self) -> usize {
            match self {
                GgmlType::F32 | GgmlType::F16 | GgmlType::BF16 => 1,
                GgmlType::Q8_0 => 32,
                GgmlType::Q4_K | GgmlType::Q6_K => 256,
            }
        }
        pub fn type_size(self) -> usize {
            match self {
                GgmlType::F32 => 4,
                GgmlType::F16 | GgmlType::BF16 => 2,
                GgmlType::Q8_0 => 34,
                GgmlType::Q4_K => 144,
                GgmlType::Q6_K => 210,
            }
        }
    }

    /// types.rs:5-15, plus the HIP failures the reference cannot have.
    #[derive(Debug, Clone, PartialEq, Eq)]
    pub enum QuantError {
        UnsupportedType(u32),
        BufferTooSmall { expected: usize, actual: usize },
        DimensionMisaligned { dim: usize, block_size: usize },
        ArithmeticOverflow,
        Device(i32, String),
    }

    impl std::fmt::Display for QuantError {
        fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
            match self {
                QuantError::UnsupportedType(t) => write!(f, "Unsupported GGML type: {t}"),
                QuantError::BufferTooSmall { expected, actual } => {
                    write!(f, "Buffer too small: expected {expected}, got {actual}")
                }
                QuantError::DimensionMisaligned { dim, block_size } => {
                    write!(f, "Dimension {dim} not aligned to block size {block_size}")
                }
                QuantError::ArithmeticOverflow => write!(f, "Arithmetic overflow"),
                QuantError::Device(code, msg) => write!(f, "mivi-hip error {code}: {msg}"),
            }
        }
    }

    impl std::error::Error for QuantError {}

    pub type Result<T> = std::result::Result<T, QuantError>;

    /// A status of the C ABI as the reference's error (0 = Ok, 1..4 =
    /// QuantError in declaration order, >= 100 = device errors).
    pub fn check(rc: i32) -> Result<()> {
        if rc == ffi::MIVI_OK {
            return Ok(());
        }
        let mut e = std::mem::MaybeUninit::<ffi::MiviError>::zeroed();
        let e = unsafe {
            ffi::mivi_hip_last_error(e.as_mut_ptr());
            e.assume_init()
        };
        Err(match rc {
            ffi::MIVI_ERR_UNSUPPORTED_TYPE => QuantError::UnsupportedType(e.type_id),
            ffi::MIVI_ERR_BUFFER_TOO_SMALL => QuantError::BufferTooSmall { expected: e.expected, actual: e.actual },
            ffi::MIVI_ERR_DIMENSION_MISALIGNED => {
                QuantError::DimensionMisaligned { dim: e.dim, block_size: e.block_size }
            }
            ffi::MIVI_ERR_ARITHMETIC_OVERFLOW => QuantError::ArithmeticOverflow,
            code => {
                let msg = unsafe { std::ffi::CStr::from_ptr(e.message.as_ptr()) };
                QuantError::Device(code, msg.to_string_lossy().into_owned())
            }
        })
    }

    fn hip(rc: i32, what: &str) -> Result<()> {
        if rc == 0 {
            Ok(())
        } else {
            Err(QuantError::Device(ffi::MIVI_ERR_HIP, format!("{what} failed with hipError {rc}")))
        }
    }

    /// Device memory of `len` elements of T (hipMalloc / hipFree).
    pub struct DeviceBuffer<T: Copy> {
        ptr: *mut T,
        len: usize,
    }

    impl<T: Copy> DeviceBuffer<T> {
        pub fn new(len: usize) -> Result<Self> {
            let mut p: *mut c_void = std::ptr::null_mut();
            let bytes = len.checked_mul(std::mem::size_of::<T>()).ok_or(QuantError::ArithmeticOverflow)?;
            hip(unsafe { ffi::hipMalloc(&mut p, bytes.max(1)) }, "hipMalloc")?;
            Ok(Self { ptr: p as *mut T, len })
        }
        pub fn from_slice(src: &[T]) -> Result<Self> {
            let b = Self::new(src.len())?;
            hip(unsafe {
                ffi::hipMemcpy(b.ptr as *mut c_void, src.as_ptr() as *const c_void,
                               std::mem::size_of_val(src), ffi::HIP_MEMCPY_HOST_TO_DEVICE)
            }, "hipMemcpy")?;
            Ok(b)
        }
        pub fn copy_to(&self, dst: &mut [T]) -> Result<()> {
            let n = dst.len().min(self.len);
            hip(unsafe {
                ffi::hipMemcpy(dst.as_mut_ptr() as *mut c_void, self.ptr as *const c_void,
                               n * std::mem::size_of::<T>(), ffi::HIP_MEMCPY_DEVICE_TO_HOST)
            }, "hipMemcpy")
        }
        pub fn len(&self) -> usize {
            self.len
        }
        pub fn is_empty(&self) -> bool {
            self.len == 0
        }
        pub fn as_ptr(&self) -> *const T {
            self.ptr
        }
        pub fn as_mut_ptr(&mut self) -> *mut T {
            self.ptr
        }
    }

    impl<T: Copy> Drop for DeviceBuffer<T> {
        fn drop(&mut self) {
            unsafe {
                ffi::hipFree(self.ptr as *mut c_void);
            }
        }
    }

    /// `quantized_matvec` (lib.rs:75-134) over device-resident buffers on the
    /// default stream: out[n] = W[n, d] x[d]; asynchronous, the tail of out
    /// past n untouched.
    pub fn quantized_matvec_device(out: &mut DeviceBuffer<f32>, ggml_type: GgmlType, weights: &DeviceBuffer<u8>,
                                   x: &DeviceBuffer<f32>, n: usize, d: usize) -> Result<()> {
        check(unsafe {
            ffi::mivi_hip_quantized_matvec(out.as_mut_ptr(), out.len(), ggml_type as i32, weights.as_ptr(),
                                           weights.len(), x.as_ptr(), x.len(), n, d, std::ptr::null_mut())
        })
    }

    /// `quantized_matvec` with the reference's signature (lib.rs:75-82):
    /// host slices in and out, staged through device memory. The arguments
    /// are validated before anything is copied (types.rs:146-235), so on an
    /// error `out` is untouched.
    pub fn quantized_matvec(out: &mut [f32], ggml_type: GgmlType, weights: &[u8], x: &[f32], n: usize,
                            d: usize) -> Result<()> {
        // the library validates on the host first: a call with null device
        // pointers and the real lengths returns the reference's error without
        // launching anything
        let rc = unsafe {
            ffi::mivi_hip_quantized_matvec(std::ptr::null_mut(), out.len(), ggml_type as i32, std::ptr::null(),
                                           weights.len(), std::ptr::null(), x.len(), n, d, std::ptr::null_mut())
        };
        if rc != ffi::MIVI_ERR_INVALID_ARGUMENT {
            check(rc)?;
        }
        let w = DeviceBuffer::from_slice(weights)?;
        let xv = DeviceBuffer::from_slice(x)?;
        let mut o = DeviceBuffer::<f32>::from_slice(out)?;
        quantized_matvec_device(&mut o, ggml_type, &w, &xv, n, d)?;
        hip(unsafe { ffi::hipDeviceSynchronize() }, "hipDeviceSynchronize")?;
        o.copy_to(out)
    }

    /// `quantized_matmul_rows` with the reference's signature (lib.rs:136-151):
    /// out[batch, rows] = inputs[batch, cols] W[rows, cols]^T, staged through
    /// device memory.
    pub fn quantized_matmul_rows(out: &mut [f32], ggml_type: GgmlType, weights: &[u8], inputs: &[f32],
                                 batch: usize, rows: usize, cols: usize) -> Result<()> {
        let rc = unsafe {
            ffi::mivi_hip_quantized_matmul_rows(std::ptr::null_mut(), out.len(), ggml_type as i32,
                                                std::ptr::null(), weights.len(), std::ptr::null(), inputs.len(),
                                                batch, rows, cols, std::ptr::null_mut())
        };
        if rc != ffi::MIVI_ERR_INVALID_ARGUMENT {
            check(rc)?;
        }
        let w = DeviceBuffer::from_slice(weights)?;
        let xi = DeviceBuffer::from_slice(inputs)?;
        let mut o = DeviceBuffer::<f32>::from_slice(out)?;
        check(unsafe {
            ffi::mivi_hip_quantized_matmul_rows(o.as_mut_ptr(), o.len(), ggml_type as i32, w.as_ptr(), w.len(),
                                                xi.as_ptr(), xi.len(), batch, rows, cols, std::ptr::null_mut())
        })?;
        hip(unsafe { ffi::hipDeviceSynchronize() }, "hipDeviceSynchronize")?;
        o.copy_to(out)
    }

    /// `dequantize_slice` with the reference's signature (lib.rs:35):
    /// bit-exact decode of `bytes` into `out`.
    pub fn dequantize_slice(ggml_type: GgmlType, bytes: &[u8], out: &mut [f32]) -> Result<()> {
        let b = DeviceBuffer::from_slice(bytes)?;
        let mut o = DeviceBuffer::<f32>::new(out.len())?;
        check(unsafe {
            ffi::mivi_hip_dequantize_slice(ggml_type as i32, b.as_ptr(), b.len(), o.as_mut_ptr(), o.len(),
                                           std::ptr::null_mut())
        })?;
        hip(unsafe { ffi::hipDeviceSynchronize() }, "hipDeviceSynchronize")?;
        o.copy_to(out)
    }

    /// `try_matvec_q4_k_m` (q4_k_m.rs:217-237) with the reference's signature.
    pub fn try_matvec_q4_k_m(out: &mut [f32], weights: &[u8], x: &[f32], n: usize, d: usize) -> Result<()> {
        quantized_matvec(out, GgmlType::Q4_K, weights, x, n, d)
    }

    /// `try_matvec_q6_k` (q6_k.rs:202-221) with the reference's signature.
    pub fn try_matvec_q6_k(out: &mut [f32], weights: &[u8], x: &[f32], n: usize, d: usize) -> Result<()> {
        quantized_matvec(out, GgmlType::Q6_K, weights, x, n, d)
    }

    /// `try_matvec_q8_0` (q8_0.rs:127-147) with the reference's signature.
    pub fn try_matvec_q8_0(out: &mut [f32], weights: &[u8], x: &[f32], n: usize, d: usize) -> Result<()> {
        quantized_matvec(out, GgmlType::Q8_0, weights, x, n, d)
    }
}
