//! The C ABI of libqi_hip.so, field for field and function for function as
//! include/qi_hip.h declares it (a CPU test checks that every `qi_hip_*`
//! function of the header is declared here).
#![allow(non_camel_case_types, dead_code)]

use std::ffi::{c_char, c_void};

pub const QI_HIP_ABI_VERSION: i32 = 1;

pub const QI_HIP_OK: i32 = 0;
pub const QI_HIP_INVALID_INPUT: i32 = 1;
pub const QI_HIP_UNSUPPORTED: i32 = 2;
pub const QI_HIP_RUNTIME_ERROR: i32 = 3;

pub const QI_HIP_F32: i32 = 0;
pub const QI_HIP_Q8_0: i32 = 1;
pub const QI_HIP_Q4_0: i32 = 2;
pub const QI_HIP_Q4_K: i32 = 3;
pub const QI_HIP_Q5_K: i32 = 4;
pub const QI_HIP_Q6_K: i32 = 5;

pub const QI_HIP_LAYOUT_ROW_MAJOR: i32 = 0;
pub const QI_HIP_LAYOUT_OUTPUT_ROWS: i32 = 1;

pub const QI_HIP_MODE_AUTO: i32 = 0;
pub const QI_HIP_MODE_F32: i32 = 1;
pub const QI_HIP_MODE_EXACT: i32 = 2;
pub const QI_HIP_MODE_MFMA: i32 = 3;

/// core quantized/q8.rs:7-11
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Q8_0 {
    pub scale: f32,
    pub values: [i8; 32],
}

/// core quantized/q4.rs:7-13 (unpacked codes 0..15)
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Q4_0 {
    pub scale: f32,
    pub values: [u8; 32],
}

/// core quantized/q4.rs:72-78
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Q4K {
    pub scale: f32,
    pub min_scale: f32,
    pub scales: [u8; 12],
    pub values: [u8; 128],
}

/// core quantized/k.rs:7-14
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Q5K {
    pub scale: f32,
    pub min_scale: f32,
    pub scales: [u8; 12],
    pub high_bits: [u8; 32],
    pub values: [u8; 128],
}

/// core quantized/k.rs:55-61
#[repr(C)]
#[derive(Clone, Copy)]
pub struct Q6K {
    pub scale: f32,
    pub scales: [i8; 16],
    pub low_bits: [u8; 128],
    pub high_bits: [u8; 64],
}

#[repr(C)]
pub struct Ctx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct Weights {
    _p: [u8; 0],
}
#[repr(C)]
pub struct Qwen3 {
    _p: [u8; 0],
}
#[repr(C)]
pub struct KvCache {
    _p: [u8; 0],
}

#[repr(C)]
#[derive(Clone, Copy, Default)]
pub struct WeightsInfo {
    pub qtype: i32,
    pub layout: i32,
    pub k: u64,
    pub n: u64,
    pub device_bytes: u64,
    pub f16_scales: i32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct Qwen3Config {
    pub vocab_size: u32,
    pub hidden_size: u32,
    pub intermediate_size: u32,
    pub num_hidden_layers: u32,
    pub num_attention_heads: u32,
    pub num_key_value_heads: u32,
    pub head_dim: u32,
    pub max_position_embeddings: u32,
    pub rms_norm_eps: f32,
    pub rope_theta: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct LinearWeight {
    pub qtype: i32,
    pub layout: i32,
    pub data: *const c_void,
    pub count: u64,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct Qwen3Layer {
    pub input_layernorm: *const f32,
    pub q_norm: *const f32,
    pub k_norm: *const f32,
    pub post_attention_layernorm: *const f32,
    pub q_proj: LinearWeight,
    pub k_proj: LinearWeight,
    pub v_proj: LinearWeight,
    pub o_proj: LinearWeight,
    pub gate_proj: LinearWeight,
    pub up_proj: LinearWeight,
    pub down_proj: LinearWeight,
}

#[repr(C)]
#[derive(Clone, Copy, Default)]
pub struct Qwen3Timing {
    pub prefill_ms: f64,
    pub decode_ms: f64,
    pub prompt_tokens: u64,
    pub decode_steps: u64,
}

extern "C" {
    pub fn qi_hip_abi_version() -> i32;
    pub fn qi_hip_last_error() -> *const c_char;
    pub fn qi_hip_open(device: i32, out: *mut *mut Ctx) -> i32;
    pub fn qi_hip_close(ctx: *mut Ctx);
    pub fn qi_hip_device_name(ctx: *mut Ctx, buf: *mut c_char, len: usize) -> i32;
    pub fn qi_hip_weights_create(ctx: *mut Ctx, qtype: i32, layout: i32, k: u64, n: u64,
                                 blocks: *const c_void, count: u64, out: *mut *mut Weights) -> i32;
    pub fn qi_hip_weights_free(w: *mut Weights);
    pub fn qi_hip_weights_info_get(w: *const Weights, out: *mut WeightsInfo) -> i32;
    pub fn qi_hip_linear(ctx: *mut Ctx, w: *const Weights, x_host: *const f32, m: u64,
                         y_host: *mut f32, mode: i32) -> i32;
    pub fn qi_hip_linear_device(ctx: *mut Ctx, w: *const Weights, x_dev: *const f32, m: u64,
                                y_dev: *mut f32, mode: i32, stream: *mut c_void) -> i32;
    pub fn qi_hip_linear_device_noalloc(ctx: *mut Ctx, w: *const Weights, x_dev: *const f32, m: u64,
                                        y_dev: *mut f32, mode: i32, stream: *mut c_void) -> i32;
    pub fn qi_hip_dequantize(ctx: *mut Ctx, w: *const Weights, out_host: *mut f32) -> i32;
    pub fn qi_hip_dequantize_device(ctx: *mut Ctx, w: *const Weights, out_dev: *mut f32,
                                    stream: *mut c_void) -> i32;
    pub fn qi_hip_pack_weights(qtype: i32, layout: i32, k: u64, n: u64, blocks: *const c_void,
                               count: u64, out: *mut c_void, bytes: *mut u64, f16_scales: *mut i32) -> i32;
    pub fn qi_hip_weights_create_gguf(ctx: *mut Ctx, qtype: i32, layout: i32, k: u64, n: u64,
                                      wire: *const c_void, wire_bytes: u64, legacy: i32,
                                      out: *mut *mut Weights) -> i32;
    pub fn qi_hip_pack_gguf(qtype: i32, layout: i32, k: u64, n: u64, wire: *const c_void,
                            wire_bytes: u64, legacy: i32, out: *mut c_void, bytes: *mut u64,
                            f16_scales: *mut i32) -> i32;
    pub fn qi_hip_quantize(qtype: i32, values: *const f32, n: u64, storage_f16: i32, out: *mut c_void,
                           out_count: u64, threads: i32) -> i32;
    pub fn qi_hip_synth_normal(seed: u64, n: u64, std: f64, outlier_rate: f64, outlier_std: f64,
                               out: *mut f32, threads: i32) -> i32;

    pub fn qi_hip_qwen3_create(ctx: *mut Ctx, config: *const Qwen3Config, out: *mut *mut Qwen3) -> i32;
    pub fn qi_hip_qwen3_set_embedding(model: *mut Qwen3, embedding: *const f32) -> i32;
    pub fn qi_hip_qwen3_set_layer(model: *mut Qwen3, index: u32, layer: *const Qwen3Layer) -> i32;
    pub fn qi_hip_qwen3_set_output(model: *mut Qwen3, final_norm: *const f32,
                                   lm_head: *const LinearWeight) -> i32;
    pub fn qi_hip_qwen3_set_mode(model: *mut Qwen3, mode: i32) -> i32;
    pub fn qi_hip_qwen3_free(model: *mut Qwen3);
    pub fn qi_hip_kv_cache_create(ctx: *mut Ctx, num_layers: u32, max_sequence_length: u32,
                                  num_key_value_heads: u32, head_dim: u32, out: *mut *mut KvCache) -> i32;
    pub fn qi_hip_kv_cache_length(cache: *const KvCache, out: *mut u64) -> i32;
    pub fn qi_hip_kv_cache_reset(cache: *mut KvCache) -> i32;
    pub fn qi_hip_kv_cache_free(cache: *mut KvCache);
    pub fn qi_hip_qwen3_forward(model: *mut Qwen3, cache: *mut KvCache, tokens: *const i32, count: u64,
                                last_logits: *mut f32, next_token: *mut i32) -> i32;
    pub fn qi_hip_qwen3_generate(model: *mut Qwen3, cache: *mut KvCache, prompt: *const i32,
                                 prompt_count: u64, max_new_tokens: u64, eos_token_id: i32,
                                 out_tokens: *mut i32, out_count: *mut u64) -> i32;
    pub fn qi_hip_qwen3_last_timing(model: *const Qwen3, out: *mut Qwen3Timing) -> i32;
}
