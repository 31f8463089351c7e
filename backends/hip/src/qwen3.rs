//! GPU-resident Qwen3 decoding: the runtime's loaded model
//! (`Qwen3LayerWeights`, crates/quantinfer-runtime/src/qwen3/mod.rs:10-22)
//! handed to the library's decoder once, then greedy generation
//! (`generate_qwen3_stream` with temperature 0, runtime/src/generation.rs:
//! 160-201) with the KV cache on the device; only token ids cross PCIe.
use std::sync::Arc;

use quantinfer_core::Tensor;
use quantinfer_kernel::{KernelError, Result};
use quantinfer_model::Qwen3Config;
use quantinfer_runtime::{LinearWeight, Qwen3LayerWeights};

use crate::{ffi, status, Context, HipBackend};

/// A loaded decoder on the device.
pub struct HipQwen3 {
    _ctx: Arc<Context>,
    raw: *mut ffi::Qwen3,
    layers: usize,
    kv_heads: u32,
    head_dim: u32,
}
unsafe impl Send for HipQwen3 {}
unsafe impl Sync for HipQwen3 {}

impl Drop for HipQwen3 {
    fn drop(&mut self) {
        unsafe { ffi::qi_hip_qwen3_free(self.raw) }
    }
}

/// A device KV cache (`KvCache::new`, runtime/src/cache.rs:25-60).
pub struct HipKvCache {
    raw: *mut ffi::KvCache,
}
unsafe impl Send for HipKvCache {}
impl Drop for HipKvCache {
    fn drop(&mut self) {
        unsafe { ffi::qi_hip_kv_cache_free(self.raw) }
    }
}

impl HipKvCache {
    pub fn len(&self) -> Result<usize> {
        let mut n = 0u64;
        status(unsafe { ffi::qi_hip_kv_cache_length(self.raw, &mut n) })?;
        Ok(n as usize)
    }

    pub fn reset(&mut self) -> Result<()> {
        status(unsafe { ffi::qi_hip_kv_cache_reset(self.raw) })
    }
}

/// The (qtype, layout, logical blocks) of a runtime linear weight; the block
/// structs are copied field for field into the C layout.
struct Linear {
    raw: ffi::LinearWeight,
    _keep: Vec<u8>,
}

fn copy_blocks<B, C>(blocks: &[B], convert: impl Fn(&B) -> C) -> Vec<u8> {
    let logical: Vec<C> = blocks.iter().map(convert).collect();
    let bytes = std::mem::size_of_val(logical.as_slice());
    let mut out = vec![0u8; bytes];
    unsafe { std::ptr::copy_nonoverlapping(logical.as_ptr().cast::<u8>(), out.as_mut_ptr(), bytes) };
    out
}

fn linear(w: &LinearWeight) -> Result<Linear> {
    use ffi::{QI_HIP_LAYOUT_OUTPUT_ROWS as OR, QI_HIP_LAYOUT_ROW_MAJOR as RM};
    let (qtype, layout, keep, count) = match w {
        LinearWeight::F32(t) => {
            let v = t.as_f32()?;
            (ffi::QI_HIP_F32, RM, copy_blocks(v, |x| *x), v.len())
        }
        LinearWeight::Q8_0(t) => (ffi::QI_HIP_Q8_0, RM, copy_blocks(t.blocks(), crate::q8), t.blocks().len()),
        LinearWeight::Q8_0OutputRows(t) => (ffi::QI_HIP_Q8_0, OR, copy_blocks(t.blocks(), crate::q8), t.blocks().len()),
        LinearWeight::Q4_0(t) => (ffi::QI_HIP_Q4_0, RM, copy_blocks(t.blocks(), crate::q4), t.blocks().len()),
        LinearWeight::Q4_0OutputRows(t) => (ffi::QI_HIP_Q4_0, OR, copy_blocks(t.blocks(), crate::q4), t.blocks().len()),
        LinearWeight::Q4_K(t) => (ffi::QI_HIP_Q4_K, RM, copy_blocks(t.blocks(), crate::q4k), t.blocks().len()),
        LinearWeight::Q4_KOutputRows(t) => (ffi::QI_HIP_Q4_K, OR, copy_blocks(t.blocks(), crate::q4k), t.blocks().len()),
        LinearWeight::Q5_K(t) => (ffi::QI_HIP_Q5_K, RM, copy_blocks(t.blocks(), crate::q5k), t.blocks().len()),
        LinearWeight::Q5_KOutputRows(t) => (ffi::QI_HIP_Q5_K, OR, copy_blocks(t.blocks(), crate::q5k), t.blocks().len()),
        LinearWeight::Q6_K(t) => (ffi::QI_HIP_Q6_K, RM, copy_blocks(t.blocks(), crate::q6k), t.blocks().len()),
        LinearWeight::Q6_KOutputRows(t) => (ffi::QI_HIP_Q6_K, OR, copy_blocks(t.blocks(), crate::q6k), t.blocks().len()),
        LinearWeight::Lora { .. } => {
            return Err(KernelError::Unsupported("HIP decoder: LoRA projections are not supported".into()))
        }
    };
    Ok(Linear {
        raw: ffi::LinearWeight { qtype, layout, data: keep.as_ptr().cast(), count: count as u64 },
        _keep: keep,
    })
}

fn f32s(t: &Tensor) -> Result<&[f32]> {
    Ok(t.as_f32()?)
}

impl HipQwen3 {
    /// Upload a loaded model: embedding [vocab, hidden] f32, the layers, the
    /// final norm and the LM head ([hidden, vocab]; a Q6_K output-rows head
    /// stays quantized on the device).
    pub fn new(backend: &HipBackend, config: &Qwen3Config, embedding: &Tensor,
               layers: &[Qwen3LayerWeights], final_norm: &Tensor, lm_head: &LinearWeight) -> Result<Self> {
        let cfg = ffi::Qwen3Config {
            vocab_size: config.vocab_size as u32,
            hidden_size: config.hidden_size as u32,
            intermediate_size: config.intermediate_size as u32,
            num_hidden_layers: config.num_hidden_layers as u32,
            num_attention_heads: config.num_attention_heads as u32,
            num_key_value_heads: config.num_key_value_heads as u32,
            head_dim: config.effective_head_dim() as u32,
            max_position_embeddings: config.max_position_embeddings as u32,
            rms_norm_eps: config.rms_norm_eps,
            rope_theta: config.rope_theta,
        };
        let mut raw = std::ptr::null_mut();
        status(unsafe { ffi::qi_hip_qwen3_create(backend.ctx.0, &cfg, &mut raw) })?;
        let model = Self { _ctx: backend.ctx.clone(), raw, layers: layers.len(),
                           kv_heads: cfg.num_key_value_heads, head_dim: cfg.head_dim };
        status(unsafe { ffi::qi_hip_qwen3_set_embedding(raw, f32s(embedding)?.as_ptr()) })?;
        for (i, l) in layers.iter().enumerate() {
            let p = [&l.q_proj, &l.k_proj, &l.v_proj, &l.o_proj, &l.gate_proj, &l.up_proj, &l.down_proj]
                .map(linear);
            let [q, k, v, o, g, u, d] = p;
            let (q, k, v, o, g, u, d) = (q?, k?, v?, o?, g?, u?, d?);
            let layer = ffi::Qwen3Layer {
                input_layernorm: f32s(&l.input_layernorm)?.as_ptr(),
                q_norm: f32s(&l.q_norm)?.as_ptr(),
                k_norm: f32s(&l.k_norm)?.as_ptr(),
                post_attention_layernorm: f32s(&l.post_attention_layernorm)?.as_ptr(),
                q_proj: q.raw, k_proj: k.raw, v_proj: v.raw, o_proj: o.raw,
                gate_proj: g.raw, up_proj: u.raw, down_proj: d.raw,
            };
            status(unsafe { ffi::qi_hip_qwen3_set_layer(raw, i as u32, &layer) })?;
        }
        let head = linear(lm_head)?;
        status(unsafe { ffi::qi_hip_qwen3_set_output(raw, f32s(final_norm)?.as_ptr(), &head.raw) })?;
        Ok(model)
    }

    /// QI_HIP_MODE_* for every linear layer (default AUTO).
    pub fn set_mode(&self, mode: i32) -> Result<()> {
        status(unsafe { ffi::qi_hip_qwen3_set_mode(self.raw, mode) })
    }

    pub fn kv_cache(&self, backend: &HipBackend, max_sequence_length: usize) -> Result<HipKvCache> {
        let mut raw = std::ptr::null_mut();
        status(unsafe {
            ffi::qi_hip_kv_cache_create(backend.ctx.0, self.layers as u32, max_sequence_length as u32,
                                        self.kv_heads, self.head_dim, &mut raw)
        })?;
        Ok(HipKvCache { raw })
    }

    /// `Qwen3Model::forward` for the last row: its logits ([vocab]) and argmax.
    pub fn forward(&self, cache: &mut HipKvCache, tokens: &[usize], logits: Option<&mut [f32]>)
                   -> Result<usize> {
        let ids: Vec<i32> = tokens.iter().map(|&t| t as i32).collect();
        let mut next = 0i32;
        let out = logits.map_or(std::ptr::null_mut(), |l| l.as_mut_ptr());
        status(unsafe {
            ffi::qi_hip_qwen3_forward(self.raw, cache.raw, ids.as_ptr(), ids.len() as u64, out, &mut next)
        })?;
        Ok(next as usize)
    }

    /// Greedy generation: the prompt, then up to `max_new` argmax steps or the
    /// EOS id; one call, the decode steps replayed on the device.
    pub fn generate(&self, cache: &mut HipKvCache, prompt: &[usize], max_new: usize,
                    eos: Option<usize>) -> Result<Vec<usize>> {
        let ids: Vec<i32> = prompt.iter().map(|&t| t as i32).collect();
        let mut out = vec![0i32; max_new.max(1)];
        let mut count = 0u64;
        status(unsafe {
            ffi::qi_hip_qwen3_generate(self.raw, cache.raw, ids.as_ptr(), ids.len() as u64, max_new as u64,
                                       eos.map_or(-1, |e| e as i32), out.as_mut_ptr(), &mut count)
        })?;
        Ok(out[..count as usize].iter().map(|&t| t as usize).collect())
    }
}
