//! QuantInfer backend for AMD Instinct MI355X (gfx950): the quantized-linear
//! methods of `KernelBackend` (crates/quantinfer-kernel/src/lib.rs:83-154) on
//! hand-written HIP kernels, through the C ABI of libqi_hip.so
//! (include/qi_hip.h, bound in `ffi`). The other operators stay on the CPU
//! reference, as in backends/cuda/src/native.rs:185-207.
//!
//! Weights are uploaded once and kept resident: a handle per (block slice
//! address, block count, K*N, layout), since a loaded model's weights are
//! immutable. Each matmul call copies the activations in and the outputs back
//! (`qi_hip_linear`, synchronous), the same contract as `CpuScalar`.
//!
//! This crate is not compiled in the environment it was written in (no cargo
//! there); the C ABI it binds is the tested boundary.

mod ffi;
pub mod qwen3;

use std::collections::HashMap;
use std::ffi::CStr;
use std::sync::{Arc, Mutex};

use quantinfer_backend_cpu::CpuScalar;
use quantinfer_core::{
    QuantizedTensor, QuantizedTensor4, QuantizedTensorQ4K, QuantizedTensorQ5K, QuantizedTensorQ6K,
    Tensor,
};
use quantinfer_gpu_common::projection_capabilities;
use quantinfer_kernel::{BackendId, KernelBackend, KernelError, Result};
use quantinfer_runtime::{KernelCapability, RuntimeProvider};

pub use ffi::{QI_HIP_MODE_AUTO, QI_HIP_MODE_EXACT, QI_HIP_MODE_F32, QI_HIP_MODE_MFMA};

pub(crate) struct Handle(*mut ffi::Weights);
// A weights handle is an immutable device image; the library serializes calls.
unsafe impl Send for Handle {}
unsafe impl Sync for Handle {}
impl Drop for Handle {
    fn drop(&mut self) {
        unsafe { ffi::qi_hip_weights_free(self.0) }
    }
}

pub(crate) struct Context(pub(crate) *mut ffi::Ctx);
// Calls on one context are serialized by the library's mutex.
unsafe impl Send for Context {}
unsafe impl Sync for Context {}
impl Drop for Context {
    fn drop(&mut self) {
        // weights handles hold their own reference: close and free may come in any order
        unsafe { ffi::qi_hip_close(self.0) }
    }
}

type CacheKey = (usize, usize, usize, i32, i32);

/// Projections on one MI355X.
#[derive(Clone)]
pub struct HipBackend {
    ctx: Arc<Context>,
    cache: Arc<Mutex<HashMap<CacheKey, Arc<Handle>>>>,
    mode: i32,
    name: String,
    capabilities: Vec<KernelCapability>,
    cpu: CpuScalar,
}

impl std::fmt::Debug for HipBackend {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        f.debug_struct("HipBackend").field("name", &self.name).field("mode", &self.mode).finish()
    }
}

/// Map a library status to the reference's errors: INVALID_INPUT ->
/// InvalidInput; UNSUPPORTED and RUNTIME_ERROR -> Unsupported (the mapping
/// backends/cuda/src/native.rs:238-244 uses for device failures).
pub(crate) fn status(code: i32) -> Result<()> {
    if code == ffi::QI_HIP_OK {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(ffi::qi_hip_last_error()) }.to_string_lossy().into_owned();
    Err(if code == ffi::QI_HIP_INVALID_INPUT {
        KernelError::InvalidInput(format!("HIP {msg}"))
    } else {
        KernelError::Unsupported(format!("HIP {msg}"))
    })
}

impl HipBackend {
    /// Open HIP device `ordinal` (gfx950 only) with the F32 arithmetic mode:
    /// every linear within 1e-5 of the CPU result at any row count (f32 GEMV
    /// kernels; for prompts of 48+ rows a matrix-core GEMM of exact
    /// products), so greedy ids equal a CPU run's
    /// (runtime/src/generation.rs:58-76).
    pub fn open(ordinal: usize) -> Result<Self> {
        Self::open_with_mode(ordinal, ffi::QI_HIP_MODE_F32)
    }

    /// `mode`: QI_HIP_MODE_EXACT reproduces CpuScalar bit for bit;
    /// QI_HIP_MODE_AUTO prefills 128+ rows on the f16-operand GEMM (faster
    /// prompts, within 2e-3 normwise of the CPU result).
    pub fn open_with_mode(ordinal: usize, mode: i32) -> Result<Self> {
        if unsafe { ffi::qi_hip_abi_version() } != ffi::QI_HIP_ABI_VERSION {
            return Err(KernelError::Unsupported("HIP library ABI version mismatch".into()));
        }
        let device = i32::try_from(ordinal)
            .map_err(|_| KernelError::Unsupported("HIP device ordinal out of range".into()))?;
        let mut raw = std::ptr::null_mut();
        status(unsafe { ffi::qi_hip_open(device, &mut raw) })?;
        let ctx = Arc::new(Context(raw));
        let mut buf = [0 as std::ffi::c_char; 256];
        status(unsafe { ffi::qi_hip_device_name(ctx.0, buf.as_mut_ptr(), buf.len()) })?;
        let name = unsafe { CStr::from_ptr(buf.as_ptr()) }.to_string_lossy().into_owned();
        Ok(Self {
            ctx,
            cache: Default::default(),
            mode,
            name,
            // F32, Q8_0 and Q4_0 in both layouts (gpu-common lib.rs:84-117); the
            // K-quant methods below also run on the device
            capabilities: projection_capabilities(),
            cpu: CpuScalar::new(),
        })
    }

    pub fn device_name(&self) -> &str {
        &self.name
    }

    /// Upload once per (blocks pointer, block count, K*N, qtype, layout).
    fn resident<B, C>(&self, qtype: i32, layout: i32, k: usize, n: usize, blocks: &[B],
                      convert: impl Fn(&B) -> C) -> Result<Arc<Handle>> {
        let key = (blocks.as_ptr() as usize, blocks.len(), k * n, qtype, layout);
        if let Some(h) = self.cache.lock().unwrap().get(&key) {
            return Ok(h.clone());
        }
        let logical: Vec<C> = blocks.iter().map(convert).collect();
        let mut w = std::ptr::null_mut();
        status(unsafe {
            ffi::qi_hip_weights_create(self.ctx.0, qtype, layout, k as u64, n as u64,
                                       logical.as_ptr().cast(), logical.len() as u64, &mut w)
        })?;
        let h = Arc::new(Handle(w));
        self.cache.lock().unwrap().insert(key, h.clone());
        Ok(h)
    }

    fn linear(&self, lhs: &Tensor, w: &Handle, n: usize) -> Result<Tensor> {
        let &[m, _k] = lhs.shape().dims() else {
            return Err(KernelError::InvalidInput("HIP left matrix must have rank 2".into()));
        };
        let x = lhs.as_f32()?;
        let mut y = vec![0.0f32; m * n];
        status(unsafe {
            ffi::qi_hip_linear(self.ctx.0, w.0, x.as_ptr(), m as u64, y.as_mut_ptr(), self.mode)
        })?;
        Ok(Tensor::from_f32(vec![m, n], y)?)
    }
}

fn kn(shape: &quantinfer_core::Shape) -> Result<(usize, usize)> {
    match shape.dims() {
        &[k, n] => Ok((k, n)),
        _ => Err(KernelError::InvalidInput("HIP quantized matrix must have rank 2".into())),
    }
}

fn q8(b: &quantinfer_core::Q8_0Block) -> ffi::Q8_0 {
    ffi::Q8_0 { scale: b.scale, values: b.values }
}
fn q4(b: &quantinfer_core::Q4_0Block) -> ffi::Q4_0 {
    ffi::Q4_0 { scale: b.scale, values: b.values }
}
fn q4k(b: &quantinfer_core::Q4KBlock) -> ffi::Q4K {
    ffi::Q4K { scale: b.scale, min_scale: b.min_scale, scales: b.scales, values: b.values }
}
fn q5k(b: &quantinfer_core::Q5KBlock) -> ffi::Q5K {
    ffi::Q5K { scale: b.scale, min_scale: b.min_scale, scales: b.scales, high_bits: b.high_bits,
               values: b.values }
}
fn q6k(b: &quantinfer_core::Q6KBlock) -> ffi::Q6K {
    ffi::Q6K { scale: b.scale, scales: b.scales, low_bits: b.low_bits, high_bits: b.high_bits }
}

macro_rules! quantized {
    ($name:ident, $tensor:ty, $qtype:expr, $layout:expr, $conv:expr) => {
        fn $name(&self, lhs: &Tensor, rhs: &$tensor) -> Result<Tensor> {
            let (k, n) = kn(rhs.shape())?;
            let h = self.resident($qtype, $layout, k, n, rhs.blocks(), $conv)?;
            self.linear(lhs, &h, n)
        }
    };
}

impl RuntimeProvider for HipBackend {
    fn name(&self) -> &str {
        "hip"
    }

    fn capabilities(&self) -> &[KernelCapability] {
        &self.capabilities
    }
}

impl KernelBackend for HipBackend {
    fn backend_id(&self) -> Option<BackendId> {
        Some(BackendId::Hip)
    }

    fn reuse_workspace(&self) -> bool {
        self.cpu.reuse_workspace()
    }

    fn matmul(&self, lhs: &Tensor, rhs: &Tensor) -> Result<Tensor> {
        let (k, n) = kn(rhs.shape())?;
        let w = rhs.as_f32()?;
        let h = self.resident(ffi::QI_HIP_F32, ffi::QI_HIP_LAYOUT_ROW_MAJOR, k, n, w, |v| *v)?;
        self.linear(lhs, &h, n)
    }

    quantized!(matmul_q8_0, QuantizedTensor, ffi::QI_HIP_Q8_0, ffi::QI_HIP_LAYOUT_ROW_MAJOR, q8);
    quantized!(matmul_q4_0, QuantizedTensor4, ffi::QI_HIP_Q4_0, ffi::QI_HIP_LAYOUT_ROW_MAJOR, q4);
    quantized!(matmul_q8_0_output_rows, QuantizedTensor, ffi::QI_HIP_Q8_0,
               ffi::QI_HIP_LAYOUT_OUTPUT_ROWS, q8);
    quantized!(matmul_q4_0_output_rows, QuantizedTensor4, ffi::QI_HIP_Q4_0,
               ffi::QI_HIP_LAYOUT_OUTPUT_ROWS, q4);
    quantized!(matmul_q4_k, QuantizedTensorQ4K, ffi::QI_HIP_Q4_K, ffi::QI_HIP_LAYOUT_ROW_MAJOR, q4k);
    quantized!(matmul_q5_k, QuantizedTensorQ5K, ffi::QI_HIP_Q5_K, ffi::QI_HIP_LAYOUT_ROW_MAJOR, q5k);
    quantized!(matmul_q6_k, QuantizedTensorQ6K, ffi::QI_HIP_Q6_K, ffi::QI_HIP_LAYOUT_ROW_MAJOR, q6k);
    quantized!(matmul_q4_k_output_rows, QuantizedTensorQ4K, ffi::QI_HIP_Q4_K,
               ffi::QI_HIP_LAYOUT_OUTPUT_ROWS, q4k);
    quantized!(matmul_q5_k_output_rows, QuantizedTensorQ5K, ffi::QI_HIP_Q5_K,
               ffi::QI_HIP_LAYOUT_OUTPUT_ROWS, q5k);
    quantized!(matmul_q6_k_output_rows, QuantizedTensorQ6K, ffi::QI_HIP_Q6_K,
               ffi::QI_HIP_LAYOUT_OUTPUT_ROWS, q6k);

    fn rms_norm(&self, input: &Tensor, weight: &Tensor, epsilon: f32) -> Result<Tensor> {
        self.cpu.rms_norm(input, weight, epsilon)
    }

    fn rms_norm_heads(&self, input: &Tensor, weight: &Tensor, epsilon: f32) -> Result<Tensor> {
        self.cpu.rms_norm_heads(input, weight, epsilon)
    }

    fn softmax(&self, input: &Tensor) -> Result<Tensor> {
        self.cpu.softmax(input)
    }

    fn silu_mul(&self, gate: &Tensor, up: &Tensor) -> Result<Tensor> {
        self.cpu.silu_mul(gate, up)
    }

    fn apply_rope(&self, input: &Tensor, cos: &[f32], sin: &[f32]) -> Result<Tensor> {
        self.cpu.apply_rope(input, cos, sin)
    }

    fn embedding(&self, table: &Tensor, token_ids: &[usize]) -> Result<Tensor> {
        self.cpu.embedding(table, token_ids)
    }
}
