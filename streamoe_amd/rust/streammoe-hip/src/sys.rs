//! Raw bindings of libsmoe's C ABI: `include/smoe.h`, one to one (names,
//! argument order and types, return types). `tests/test_rust_crate.py`
//! checks this file against the header. Status codes: 0 = SMOE_OK, else
//! SMOE_ERR_* (smoe_strerror gives the text).
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

pub const SMOE_MAX_K: u32 = 16;
pub const SMOE_ABI_VERSION: u32 = 2;

pub const SMOE_OK: c_int = 0;
pub const SMOE_ERR_INVALID_ARG: c_int = 1;
pub const SMOE_ERR_BAD_K: c_int = 2;
pub const SMOE_ERR_IN_DIM_NOT_MULTIPLE: c_int = 3;
pub const SMOE_ERR_UNSUPPORTED_BITS: c_int = 4;
pub const SMOE_ERR_UNSUPPORTED_GROUP: c_int = 5;
pub const SMOE_ERR_UNSUPPORTED_SHAPE: c_int = 6;
pub const SMOE_ERR_MISALIGNED: c_int = 7;
pub const SMOE_ERR_SCRATCH_TOO_SMALL: c_int = 8;
pub const SMOE_ERR_WORKSPACE_TOO_SMALL: c_int = 9;
pub const SMOE_ERR_HIP: c_int = 10;
pub const SMOE_ERR_NO_DEVICE: c_int = 11;
pub const SMOE_ERR_DEVICE_TIMEOUT: c_int = 12;
pub const SMOE_ERR_IO: c_int = 13;

pub const SMOE_OPT_DECODE_PATH: c_int = 1;
pub const SMOE_OPT_TRACE_BUFFER: c_int = 2;
pub const SMOE_OPT_PREFILL_GEMM: c_int = 3;

/// Opaque handle (`smoe_handle`).
#[repr(C)]
pub struct smoe_handle {
    _private: [u8; 0],
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct smoe_qweights {
    pub base: *const c_void,
    pub packed_offset: u64,
    pub scales_offset: u64,
    pub biases_offset: u64,
    pub group_size: u32,
    pub bits: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct smoe_expert_shape {
    pub hidden: u32,
    pub inter: u32,
    pub group: u32,
    pub bits: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct smoe_binding {
    pub base: *const c_void,
    pub offset: u64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct smoe_layer {
    pub shape: smoe_expert_shape,
    pub experts: *const c_void,
    pub stride: u64,
    pub n_experts: u32,
    pub k: u32,
    pub normalize: i32,
    pub router_w: *const f32,
    pub shared_expert: *const c_void,
    pub shared_gate: *const f32,
    pub router_q: *const smoe_qweights,
    pub shared_gate_q: *const smoe_qweights,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct smoe_file_layout {
    pub bits: u32,
    pub reserved: u32,
    pub expert_size: u64,
    pub stride: u64,
}

extern "C" {
    pub fn smoe_strerror(status: c_int) -> *const c_char;
    pub fn smoe_abi_version() -> u32;
    pub fn smoe_create(device: c_int, stream: *mut c_void, out: *mut *mut smoe_handle) -> c_int;
    pub fn smoe_destroy(h: *mut smoe_handle) -> c_int;
    pub fn smoe_set_stream(h: *mut smoe_handle, stream: *mut c_void) -> c_int;
    pub fn smoe_reserve(h: *mut smoe_handle, max_hidden: u32, max_inter: u32, max_experts: u32) -> c_int;
    pub fn smoe_sync(h: *mut smoe_handle) -> c_int;
    pub fn smoe_set_option(h: *mut smoe_handle, option: c_int, value: i64) -> c_int;
    pub fn smoe_qmv(h: *mut smoe_handle, w: *const smoe_qweights, x: *const f32, y: *mut f32, out_dim: u32,
                    in_dim: u32) -> c_int;
    pub fn smoe_argmax(h: *mut smoe_handle, v: *const f32, n: u32, out_index: *mut i32) -> c_int;
    pub fn smoe_qmv_argmax(h: *mut smoe_handle, w: *const smoe_qweights, x: *const f32, y: *mut f32,
                           out_dim: u32, in_dim: u32, out_index: *mut i32) -> c_int;
    pub fn smoe_qmm_workspace_size(in_dim: u32, group: u32, n_tokens: u32) -> u64;
    pub fn smoe_qmm(h: *mut smoe_handle, w: *const smoe_qweights, x: *const f32, y: *mut f32, out_dim: u32,
                    in_dim: u32, n_tokens: u32, workspace: *mut c_void, workspace_bytes: u64) -> c_int;
    pub fn smoe_dequant(h: *mut smoe_handle, w: *const smoe_qweights, in_dim: u32, row0: u32, n_rows: u32,
                        out: *mut f32) -> c_int;
    pub fn smoe_router(h: *mut smoe_handle, router_w: *const f32, x: *const f32, n_tokens: u32, n_experts: u32,
                       hidden: u32, k: u32, normalize: c_int, idx: *mut i32, weights: *mut f32,
                       logits_out: *mut f32) -> c_int;
    pub fn smoe_softmax_topk(h: *mut smoe_handle, logits: *const f32, n_tokens: u32, n_experts: u32, k: u32,
                             normalize: c_int, idx: *mut i32, weights: *mut f32) -> c_int;
    pub fn smoe_softmax(h: *mut smoe_handle, logits: *const f32, n_tokens: u32, n: u32, probs: *mut f32) -> c_int;
    pub fn smoe_expf(h: *mut smoe_handle, x: *const f32, y: *mut f32, n: u64) -> c_int;
    pub fn smoe_topk(h: *mut smoe_handle, scores: *const f32, n_tokens: u32, n: u32, k: u32, idx: *mut i32,
                     values: *mut f32) -> c_int;
    pub fn smoe_noaux_tc_topk(h: *mut smoe_handle, logits: *const f32, correction_bias: *const f32,
                              n_tokens: u32, n_experts: u32, n_group: u32, topk_group: u32, k: u32,
                              routed_scaling_factor: f32, idx: *mut i32, weights: *mut f32,
                              scores_out: *mut f32) -> c_int;
    pub fn smoe_expert_bytes(shape: *const smoe_expert_shape) -> u64;
    pub fn smoe_experts_decode(h: *mut smoe_handle, shape: *const smoe_expert_shape,
                               bindings: *const smoe_binding, k: u32, weights: *const f32, input: *const f32,
                               h_mid: *const f32, shared_out: *const f32, shared_gate_score: f32,
                               hidden_out: *mut f32) -> c_int;
    pub fn smoe_moe_decode_layer(h: *mut smoe_handle, layer: *const smoe_layer, input: *const f32,
                                 h_mid: *const f32, hidden_out: *mut f32, idx_out: *mut i32,
                                 w_out: *mut f32) -> c_int;
    pub fn smoe_moe_decode_layers(h: *mut smoe_handle, layers: *const smoe_layer, n_layers: u32,
                                  norm_w: *const *const c_void, eps: f32, input: *const f32,
                                  residual_io: *mut f32, work: *mut f32) -> c_int;
    pub fn smoe_moe_decode_layers_noalloc(stream: *mut c_void, layers: *const smoe_layer, n_layers: u32,
                                          norm_w: *const *const c_void, eps: f32, input: *const f32,
                                          residual_io: *mut f32) -> c_int;
    pub fn smoe_moe_decode_tokens(h: *mut smoe_handle, layers: *const smoe_layer, n_layers: u32,
                                  norm_w: *const *const c_void, eps: f32, n_tokens: u32, input: *const f32,
                                  residual_io: *mut f32, work: *mut f32, idx_out: *mut i32,
                                  w_out: *mut f32) -> c_int;
    pub fn smoe_moe_prefill_workspace_size(shape: *const smoe_expert_shape, n_tokens: u32, n_experts: u32,
                                           k: u32) -> u64;
    pub fn smoe_moe_prefill(h: *mut smoe_handle, shape: *const smoe_expert_shape, experts: *const c_void,
                            stride: u64, n_experts: u32, idx: *const i32, weights: *const f32,
                            x: *const c_void, x_is_bf16: c_int, n_tokens: u32, k: u32, out_sum: *mut f32,
                            workspace: *mut c_void, workspace_bytes: u64) -> c_int;
    pub fn smoe_moe_prefill_block_workspace_size(shape: *const smoe_expert_shape, n_tokens: u32, n_experts: u32,
                                                 k: u32, has_shared: c_int) -> u64;
    pub fn smoe_moe_prefill_block(h: *mut smoe_handle, shape: *const smoe_expert_shape, experts: *const c_void,
                                  stride: u64, n_experts: u32, idx: *const i32, weights: *const f32,
                                  x: *const c_void, x_is_bf16: c_int, n_tokens: u32, k: u32,
                                  shared_expert: *const c_void, shared_gate: *const f32, h_mid: *const f32,
                                  hidden_out: *mut f32, workspace: *mut c_void, workspace_bytes: u64) -> c_int;
    pub fn smoe_layer_file_layout(file_bytes: u64, n_experts: u32, hidden: u32, inter: u32, group: u32,
                                  declared_size: u64, declared_stride: u64,
                                  out: *mut smoe_file_layout) -> c_int;
    pub fn smoe_load_file(h: *mut smoe_handle, path: *const c_char, offset: u64, bytes: u64, dst: *mut c_void,
                          dst_bytes: u64, bytes_read: *mut u64) -> c_int;
    pub fn smoe_stream_read(h: *mut smoe_handle, buf: *const c_void, bytes: u64, sink: *mut u32) -> c_int;
    pub fn smoe_synth_experts(h: *mut smoe_handle, base: *mut c_void, n_experts: u32, stride: u64,
                              shape: *const smoe_expert_shape, seed: u64, scale_sigma: f32,
                              bias_sigma: f32) -> c_int;
    pub fn smoe_synth_normal_f32(h: *mut smoe_handle, out: *mut f32, n: u64, seed: u64, sigma: f32) -> c_int;
    pub fn smoe_synth_normal_bf16(h: *mut smoe_handle, out: *mut u16, n: u64, seed: u64, sigma: f32) -> c_int;
}
