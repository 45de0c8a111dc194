//! streammoe-hip: the MI355X backend of streammoe's routed-expert path.
//!
//! The engine keeps its MoE encoders and calls this crate where it called
//! `streammoe_metal` (crates/streammoe-metal/src/lib.rs): [`Kernels::new`]
//! replaces `Kernels::new` (lib.rs:542-665), [`Kernels::encode`] with a
//! [`KernelCall`] replaces `Kernels::encode` (lib.rs:667-676, trait at
//! 472-482), and the call structs carry the same bindings as the Metal ones
//! (`QuantWeights` lib.rs:339-351, `QmmCall` 363-380, the `(&Buffer, u64)`
//! expert bindings of expert_forward.rs:927-986). A Metal buffer becomes a
//! device allocation ([`BufferRef`]); a command buffer becomes the handle's
//! HIP stream: every call only enqueues, [`Kernels::sync`] waits. Where the
//! Metal crate panics on an unsupported group, width or k, these calls
//! return [`SmoeError`].
//!
//! Built on `libsmoe.so` (include/smoe.h); see `sys` for the raw ABI.

pub mod sys;

use std::ffi::{CStr, CString};
use std::fmt;
use std::os::raw::{c_int, c_void};
use std::ptr;

/// A libsmoe status other than SMOE_OK, with its text.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct SmoeError {
    pub status: i32,
    pub what: &'static str,
}

impl fmt::Display for SmoeError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        // SAFETY: smoe_strerror returns a pointer to static storage.
        let text = unsafe { CStr::from_ptr(sys::smoe_strerror(self.status)) };
        write!(f, "{}: {} (status {})", self.what, text.to_string_lossy(), self.status)
    }
}

impl std::error::Error for SmoeError {}

fn check(status: c_int, what: &'static str) -> Result<(), SmoeError> {
    if status == sys::SMOE_OK {
        Ok(())
    } else {
        Err(SmoeError { status, what })
    }
}

/// A device allocation on the handle's GPU (the Metal `BufferRef`): a HIP
/// device pointer and its size in bytes. The engine owns the memory.
#[derive(Clone, Copy, Debug)]
pub struct BufferRef {
    pub ptr: *mut c_void,
    pub len: u64,
}

impl BufferRef {
    /// The address `offset` bytes into the buffer when `bytes` more bytes
    /// from there lie inside it; else `SMOE_ERR_INVALID_ARG` (checked in
    /// every build: the pointer goes to the device unverified).
    fn span(&self, offset: u64, bytes: u64, what: &'static str) -> Result<*mut c_void, SmoeError> {
        match offset.checked_add(bytes) {
            Some(end) if end <= self.len => Ok((self.ptr as *mut u8).wrapping_add(offset as usize) as *mut c_void),
            _ => Err(SmoeError { status: sys::SMOE_ERR_INVALID_ARG, what }),
        }
    }
    fn f32_span(&self, offset: u64, n: u64, what: &'static str) -> Result<*mut f32, SmoeError> {
        Ok(self.span(offset, n.checked_mul(4).unwrap_or(u64::MAX), what)? as *mut f32)
    }
}

/// A HIP stream (`hipStream_t`); null is the default stream.
#[derive(Clone, Copy, Debug)]
pub struct HipStream(pub *mut c_void);

/// MLX affine quantized weights inside one buffer (lib.rs:339-351), plus
/// the width (4, or 3 for the packed 3-bit layout).
#[derive(Clone, Copy, Debug)]
pub struct QuantWeights<'a> {
    pub buffer: &'a BufferRef,
    pub packed_offset: u64,
    pub scales_offset: u64,
    pub biases_offset: u64,
    pub group_size: u32,
    pub bits: u32,
}

/// Group sizes the quantized kernels are built for.
pub const QMM_GROUP_SIZES: &[u32] = &[64, 32, 128];

impl QuantWeights<'_> {
    /// The C view, after checking that the codes, scales and biases of an
    /// `out_dim` x `in_dim` matrix lie inside the buffer.
    fn raw(&self, out_dim: u32, in_dim: u32, what: &'static str) -> Result<sys::smoe_qweights, SmoeError> {
        let g = self.group_size.max(1) as u64;
        let codes = out_dim as u64 * in_dim as u64 * self.bits as u64 / 8;
        let sb = out_dim as u64 * (in_dim as u64 / g) * 2;
        self.buffer.span(self.packed_offset, codes, what)?;
        self.buffer.span(self.scales_offset, sb, what)?;
        self.buffer.span(self.biases_offset, sb, what)?;
        Ok(sys::smoe_qweights {
            base: self.buffer.ptr,
            packed_offset: self.packed_offset,
            scales_offset: self.scales_offset,
            biases_offset: self.biases_offset,
            group_size: self.group_size,
            bits: self.bits,
        })
    }

    /// The C view of an 8-bit router or shared gate (`rows` x `hidden`,
    /// bits 8) for [`MoeLayer::router_q8`] / [`MoeLayer::shared_gate_q8`],
    /// after the same span checks.
    pub fn rows_8bit(&self, rows: u32, hidden: u32) -> Result<sys::smoe_qweights, SmoeError> {
        if self.bits != 8 {
            return Err(SmoeError { status: sys::SMOE_ERR_UNSUPPORTED_BITS, what: "QuantWeights::rows_8bit" });
        }
        self.raw(rows, hidden, "QuantWeights::rows_8bit")
    }
}

/// The compiled kernels and their scratch on one GPU (`Kernels` +
/// `MoeBuffers`): one per engine context, `Send` but not `Sync`.
pub struct Kernels {
    h: *mut sys::smoe_handle,
}

unsafe impl Send for Kernels {}

impl Kernels {
    /// `Kernels::new`: a handle on `device` enqueueing on `stream`.
    pub fn new(device: i32, stream: HipStream) -> Result<Kernels, SmoeError> {
        // The library's struct layouts must be the ones sys.rs declares.
        // SAFETY: no arguments.
        if unsafe { sys::smoe_abi_version() } != sys::SMOE_ABI_VERSION {
            return Err(SmoeError { status: sys::SMOE_ERR_INVALID_ARG, what: "smoe_abi_version" });
        }
        let mut h = ptr::null_mut();
        // SAFETY: `h` is a valid out pointer.
        check(unsafe { sys::smoe_create(device, stream.0, &mut h) }, "smoe_create")?;
        Ok(Kernels { h })
    }

    /// Grow the decode scratch (`MoeBuffers::new_for`); allocates.
    pub fn reserve(&mut self, max_hidden: u32, max_inter: u32, max_experts: u32) -> Result<(), SmoeError> {
        check(unsafe { sys::smoe_reserve(self.h, max_hidden, max_inter, max_experts) }, "smoe_reserve")
    }

    pub fn set_stream(&mut self, stream: HipStream) -> Result<(), SmoeError> {
        check(unsafe { sys::smoe_set_stream(self.h, stream.0) }, "smoe_set_stream")
    }

    /// Wait for everything enqueued (the command buffer's commit-and-wait)
    /// and report a routing error found on the device.
    pub fn sync(&self) -> Result<(), SmoeError> {
        check(unsafe { sys::smoe_sync(self.h) }, "smoe_sync")
    }

    /// `Kernels::encode`: enqueue one call on the handle's stream.
    pub fn encode(&self, call: &impl KernelCall) -> Result<(), SmoeError> {
        call.encode(self)
    }

    /// Device workspace bytes a [`QmmCall`] needs.
    pub fn qmm_workspace_size(in_dim: u32, group: u32, n_tokens: u32) -> u64 {
        unsafe { sys::smoe_qmm_workspace_size(in_dim, group, n_tokens) }
    }

    /// Device workspace bytes a [`MoePrefillCall`] needs.
    pub fn moe_prefill_workspace_size(shape: &ExpertShape, n_tokens: u32, n_experts: u32, k: u32) -> u64 {
        let s = shape.raw();
        unsafe { sys::smoe_moe_prefill_workspace_size(&s, n_tokens, n_experts, k) }
    }

    /// Device workspace bytes a [`MoePrefillBlockCall`] needs (0: a shape
    /// the block call does not take).
    pub fn moe_prefill_block_workspace_size(shape: &ExpertShape, n_tokens: u32, n_experts: u32, k: u32,
                                            has_shared: bool) -> u64 {
        let s = shape.raw();
        unsafe { sys::smoe_moe_prefill_block_workspace_size(&s, n_tokens, n_experts, k, has_shared as c_int) }
    }

    /// Copy a byte range of a layer file into device memory (the resident
    /// part of `ExpertFiles::open` + `attach_to_device`,
    /// io/expert_io.rs:300-420); returns the bytes copied.
    pub fn load_file(&self, path: &str, offset: u64, bytes: u64, dst: &BufferRef) -> Result<u64, SmoeError> {
        let c = CString::new(path).map_err(|_| SmoeError { status: sys::SMOE_ERR_INVALID_ARG, what: "path" })?;
        let mut n = 0u64;
        check(unsafe { sys::smoe_load_file(self.h, c.as_ptr(), offset, bytes, dst.ptr, dst.len, &mut n) },
              "smoe_load_file")?;
        Ok(n)
    }
}

impl Drop for Kernels {
    fn drop(&mut self) {
        // SAFETY: `h` came from smoe_create and is released once.
        unsafe {
            sys::smoe_destroy(self.h);
        }
    }
}

/// One kernel family's parameters, encoded onto the handle's stream (the
/// Metal crate's `KernelCall`, lib.rs:472-482).
pub trait KernelCall {
    fn encode(&self, kernels: &Kernels) -> Result<(), SmoeError>;
}

/// Shape of one packed expert blob `[gate | up | down]` (variants.rs:401-486).
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct ExpertShape {
    pub hidden: u32,
    pub inter: u32,
    pub group: u32,
    pub bits: u32,
}

impl ExpertShape {
    fn raw(&self) -> sys::smoe_expert_shape {
        sys::smoe_expert_shape { hidden: self.hidden, inter: self.inter, group: self.group, bits: self.bits }
    }
    /// `expert_bytes` (variants.rs:519-528).
    pub fn expert_bytes(&self) -> u64 {
        let s = self.raw();
        unsafe { sys::smoe_expert_bytes(&s) }
    }
}

/// Single-token quantized matvec (`encode_matvec`, gpu_matvec.rs:116-159).
pub struct MatvecCall<'a> {
    pub weights: QuantWeights<'a>,
    pub input: &'a BufferRef,
    pub input_offset: u64,
    pub output: &'a BufferRef,
    pub output_offset: u64,
    pub in_dim: u32,
    pub out_dim: u32,
}

impl KernelCall for MatvecCall<'_> {
    fn encode(&self, k: &Kernels) -> Result<(), SmoeError> {
        let what = "smoe_qmv";
        let w = self.weights.raw(self.out_dim, self.in_dim, what)?;
        let x = self.input.f32_span(self.input_offset, self.in_dim as u64, what)?;
        let y = self.output.f32_span(self.output_offset, self.out_dim as u64, what)?;
        check(unsafe { sys::smoe_qmv(k.h, &w, x, y, self.out_dim, self.in_dim) }, what)
    }
}

/// Rows `[row0, row0 + n_rows)` of quantized weights (4-, 3- or 8-bit) as
/// f32 `[n_rows, in_dim]`, each weight `fma(q, s, b)` (`smoe_dequant`): the
/// load-time f32 form of an 8-bit shared-expert gate for the prefill block,
/// or a read-back for verification.
pub struct DequantCall<'a> {
    pub weights: QuantWeights<'a>,
    pub in_dim: u32,
    pub row0: u32,
    pub n_rows: u32,
    pub output: &'a BufferRef,
    pub output_offset: u64,
}

impl KernelCall for DequantCall<'_> {
    fn encode(&self, k: &Kernels) -> Result<(), SmoeError> {
        let what = "smoe_dequant";
        let rows = self.row0.checked_add(self.n_rows).ok_or(SmoeError { status: sys::SMOE_ERR_INVALID_ARG, what })?;
        let w = self.weights.raw(rows, self.in_dim, what)?;
        let out = self.output.f32_span(self.output_offset, self.n_rows as u64 * self.in_dim as u64, what)?;
        check(unsafe { sys::smoe_dequant(k.h, &w, self.in_dim, self.row0, self.n_rows, out) }, what)
    }
}

/// LM head with the greedy pick (io/gpu_lm_head.rs:130-193): logits and
/// the first index of their maximum, both left on the device.
pub struct LmHeadCall<'a> {
    pub matvec: MatvecCall<'a>,
    pub token: &'a BufferRef,
}

impl KernelCall for LmHeadCall<'_> {
    fn encode(&self, k: &Kernels) -> Result<(), SmoeError> {
        let m = &self.matvec;
        let what = "smoe_qmv_argmax";
        let w = m.weights.raw(m.out_dim, m.in_dim, what)?;
        let x = m.input.f32_span(m.input_offset, m.in_dim as u64, what)?;
        let y = m.output.f32_span(m.output_offset, m.out_dim as u64, what)?;
        let t = self.token.span(0, 4, what)? as *mut i32;
        check(unsafe { sys::smoe_qmv_argmax(k.h, &w, x, y, m.out_dim, m.in_dim, t) }, what)
    }
}

/// Dense quantized matmul (`QmmCall`, lib.rs:363-380): `output[n_tokens,
/// out_dim] = input[n_tokens, in_dim] . dequant(weights)^T`, with a
/// workspace of [`Kernels::qmm_workspace_size`] bytes.
pub struct QmmCall<'a> {
    pub weights: QuantWeights<'a>,
    pub input: &'a BufferRef,
    pub input_offset: u64,
    pub output: &'a BufferRef,
    pub output_offset: u64,
    pub in_dim: u32,
    pub out_dim: u32,
    pub n_tokens: u32,
    pub workspace: &'a BufferRef,
}

impl KernelCall for QmmCall<'_> {
    fn encode(&self, k: &Kernels) -> Result<(), SmoeError> {
        let what = "smoe_qmm";
        let w = self.weights.raw(self.out_dim, self.in_dim, what)?;
        let x = self.input.f32_span(self.input_offset, self.n_tokens as u64 * self.in_dim as u64, what)?;
        let y = self.output.f32_span(self.output_offset, self.n_tokens as u64 * self.out_dim as u64, what)?;
        check(unsafe {
            sys::smoe_qmm(k.h, &w, x, y, self.out_dim, self.in_dim, self.n_tokens, self.workspace.ptr,
                          self.workspace.len)
        }, what)
    }
}

/// Router: gate matvec, softmax, running-minimum top-k, renormalisation
/// (moe_router.rs:151-181) for `n_tokens` rows, results on the device.
pub struct RouterCall<'a> {
    pub router_w: &'a BufferRef,
    pub input: &'a BufferRef,
    pub n_tokens: u32,
    pub n_experts: u32,
    pub hidden: u32,
    pub k: u32,
    pub normalize: bool,
    pub indices: &'a BufferRef,
    pub weights: &'a BufferRef,
    pub logits: Option<&'a BufferRef>,
}

impl KernelCall for RouterCall<'_> {
    fn encode(&self, k: &Kernels) -> Result<(), SmoeError> {
        let lg = self.logits.map_or(ptr::null_mut(), |b| b.ptr as *mut f32);
        check(unsafe {
            sys::smoe_router(k.h, self.router_w.ptr as *const f32, self.input.ptr as *const f32, self.n_tokens,
                             self.n_experts, self.hidden, self.k, self.normalize as c_int,
                             self.indices.ptr as *mut i32, self.weights.ptr as *mut f32, lg)
        }, "smoe_router")
    }
}

/// K bound experts + combine for one token (`encode_experts_mmap_into`,
/// expert_forward.rs:927-986): each slot is a `(&Buffer, u64)` binding to
/// one expert blob; `weights` are host routing weights.
pub struct ExpertsDecodeCall<'a> {
    pub shape: ExpertShape,
    pub bindings: &'a [(&'a BufferRef, u64)],
    pub weights: &'a [f32],
    pub input: &'a BufferRef,
    pub h_mid: &'a BufferRef,
    pub shared_out: Option<&'a BufferRef>,
    pub shared_gate_score: f32,
    pub hidden_out: &'a BufferRef,
}

impl KernelCall for ExpertsDecodeCall<'_> {
    fn encode(&self, k: &Kernels) -> Result<(), SmoeError> {
        if self.bindings.len() != self.weights.len() || self.bindings.len() > sys::SMOE_MAX_K as usize {
            return Err(SmoeError { status: sys::SMOE_ERR_BAD_K, what: "ExpertsDecodeCall" });
        }
        let b: Vec<sys::smoe_binding> =
            self.bindings.iter().map(|(buf, off)| sys::smoe_binding { base: buf.ptr, offset: *off }).collect();
        let s = self.shape.raw();
        let so = self.shared_out.map_or(ptr::null(), |x| x.ptr as *const f32);
        check(unsafe {
            sys::smoe_experts_decode(k.h, &s, b.as_ptr(), b.len() as u32, self.weights.as_ptr(),
                                     self.input.ptr as *const f32, self.h_mid.ptr as *const f32, so,
                                     self.shared_gate_score, self.hidden_out.ptr as *mut f32)
        }, "smoe_experts_decode")
    }
}

/// One resident MoE layer (experts at `experts + e * stride`, an f32 or
/// 8-bit router, optional 4-bit shared expert with an optional f32 or 8-bit
/// gate). Exactly one of `router_w` / `router_q8` is set, at most one of
/// `shared_gate` / `shared_gate_q8` (the 8-bit forms from
/// [`QuantWeights::rows_8bit`]; A3B's mlp.gate.weight and
/// mlp.shared_expert_gate.weight, linear_attn_forward.rs:1300-1301).
#[derive(Clone, Copy, Debug)]
pub struct MoeLayer<'a> {
    pub shape: ExpertShape,
    pub experts: &'a BufferRef,
    pub stride: u64,
    pub n_experts: u32,
    pub k: u32,
    pub normalize: bool,
    pub router_w: Option<&'a BufferRef>,
    pub shared_expert: Option<&'a BufferRef>,
    pub shared_gate: Option<&'a BufferRef>,
    pub router_q8: Option<sys::smoe_qweights>,
    pub shared_gate_q8: Option<sys::smoe_qweights>,
}

impl MoeLayer<'_> {
    fn raw(&self) -> sys::smoe_layer {
        sys::smoe_layer {
            shape: self.shape.raw(),
            experts: self.experts.ptr,
            stride: self.stride,
            n_experts: self.n_experts,
            k: self.k,
            normalize: self.normalize as i32,
            router_w: self.router_w.map_or(ptr::null(), |b| b.ptr as *const f32),
            shared_expert: self.shared_expert.map_or(ptr::null(), |b| b.ptr as *const c_void),
            shared_gate: self.shared_gate.map_or(ptr::null(), |b| b.ptr as *const f32),
            // Point into self: valid while the layer is borrowed for the call.
            router_q: self.router_q8.as_ref().map_or(ptr::null(), |q| q as *const sys::smoe_qweights),
            shared_gate_q: self.shared_gate_q8.as_ref().map_or(ptr::null(), |q| q as *const sys::smoe_qweights),
        }
    }
}

/// The MoE block of one decode token with routing on the device
/// (`finish_post_attention` + `moe_dispatch_per_token`,
/// attn/linear_attn_forward.rs:2123-2165, 2382-2710).
pub struct MoeDecodeLayerCall<'a> {
    pub layer: MoeLayer<'a>,
    pub input: &'a BufferRef,
    pub h_mid: &'a BufferRef,
    pub hidden_out: &'a BufferRef,
    pub indices: Option<&'a BufferRef>,
    pub weights: Option<&'a BufferRef>,
}

impl KernelCall for MoeDecodeLayerCall<'_> {
    fn encode(&self, k: &Kernels) -> Result<(), SmoeError> {
        let l = self.layer.raw();
        check(unsafe {
            sys::smoe_moe_decode_layer(k.h, &l, self.input.ptr as *const f32, self.h_mid.ptr as *const f32,
                                       self.hidden_out.ptr as *mut f32,
                                       self.indices.map_or(ptr::null_mut(), |b| b.ptr as *mut i32),
                                       self.weights.map_or(ptr::null_mut(), |b| b.ptr as *mut f32))
        }, "smoe_moe_decode_layer")
    }
}

/// The MoE blocks of a run of layers with the next layer's RMSNorm chained
/// on the device (`ChainToNormed`, expert_forward.rs:103-111, 1317-1336):
/// layer l adds its output to `residual`, and layer l + 1 reads
/// RMSNorm(residual) * norm_w[l + 1] (bf16 weights). Capture it once into
/// a HIP graph and replay it per token (the `DeferredRing`'s role).
pub struct MoeDecodeLayersCall<'a> {
    pub layers: &'a [MoeLayer<'a>],
    pub norm_w: Option<&'a [&'a BufferRef]>,
    pub eps: f32,
    pub input: &'a BufferRef,
    pub residual: &'a BufferRef,
    pub work: &'a BufferRef,
}

impl MoeDecodeLayersCall<'_> {
    /// The C arrays; `norm_w` must have one entry per layer (the C side
    /// reads norm_w[l] for every layer).
    fn raw(&self) -> Result<(Vec<sys::smoe_layer>, Option<Vec<*const c_void>>), SmoeError> {
        if self.norm_w.is_some_and(|v| v.len() != self.layers.len()) {
            return Err(SmoeError { status: sys::SMOE_ERR_INVALID_ARG, what: "MoeDecodeLayersCall::norm_w" });
        }
        let l: Vec<sys::smoe_layer> = self.layers.iter().map(|x| x.raw()).collect();
        let n = self.norm_w.map(|v| v.iter().map(|b| b.ptr as *const c_void).collect());
        Ok((l, n))
    }

    /// The same chain without a handle or any allocation, on the current
    /// device and `stream` (smoe_moe_decode_layers_noalloc): for code under
    /// graph capture or loops that may not allocate.
    pub fn encode_noalloc(&self, stream: HipStream) -> Result<(), SmoeError> {
        let (l, n) = self.raw()?;
        let np = n.as_ref().map_or(ptr::null(), |v| v.as_ptr());
        check(unsafe {
            sys::smoe_moe_decode_layers_noalloc(stream.0, l.as_ptr(), l.len() as u32, np, self.eps,
                                                self.input.ptr as *const f32, self.residual.ptr as *mut f32)
        }, "smoe_moe_decode_layers_noalloc")
    }
}

impl KernelCall for MoeDecodeLayersCall<'_> {
    fn encode(&self, k: &Kernels) -> Result<(), SmoeError> {
        let (l, n) = self.raw()?;
        let np = n.as_ref().map_or(ptr::null(), |v| v.as_ptr());
        check(unsafe {
            sys::smoe_moe_decode_layers(k.h, l.as_ptr(), l.len() as u32, np, self.eps, self.input.ptr as *const f32,
                                        self.residual.ptr as *mut f32, self.work.ptr as *mut f32)
        }, "smoe_moe_decode_layers")
    }
}

/// Several decode tokens (1..=4) through the same layers at once
/// (`moe_dispatch_multi`, decode_multi.rs:445-654); rows are tokens.
pub struct MoeDecodeTokensCall<'a> {
    pub chain: MoeDecodeLayersCall<'a>,
    pub n_tokens: u32,
    pub indices: Option<&'a BufferRef>,
    pub weights: Option<&'a BufferRef>,
}

impl KernelCall for MoeDecodeTokensCall<'_> {
    fn encode(&self, k: &Kernels) -> Result<(), SmoeError> {
        let c = &self.chain;
        let (l, n) = c.raw()?;
        let np = n.as_ref().map_or(ptr::null(), |v| v.as_ptr());
        check(unsafe {
            sys::smoe_moe_decode_tokens(k.h, l.as_ptr(), l.len() as u32, np, c.eps, self.n_tokens,
                                        c.input.ptr as *const f32, c.residual.ptr as *mut f32,
                                        c.work.ptr as *mut f32,
                                        self.indices.map_or(ptr::null_mut(), |b| b.ptr as *mut i32),
                                        self.weights.map_or(ptr::null_mut(), |b| b.ptr as *mut f32))
        }, "smoe_moe_decode_tokens")
    }
}

/// Prefill through one layer's routed experts (`encode_moe_gather_id_fuse`,
/// expert_forward.rs:1874-2042, with `MoeIdMap0Call` / `MoeGatherIdCall` /
/// `MoeCombineTopkCall`, lib.rs:932-1189): bucketing by expert on the
/// device, grouped gate/up and down GEMMs, per-token combine into
/// `out_sum`. Workspace: [`Kernels::moe_prefill_workspace_size`] bytes.
pub struct MoePrefillCall<'a> {
    pub shape: ExpertShape,
    pub experts: &'a BufferRef,
    pub stride: u64,
    pub n_experts: u32,
    pub indices: &'a BufferRef,
    pub weights: &'a BufferRef,
    pub input: &'a BufferRef,
    pub input_is_bf16: bool,
    pub n_tokens: u32,
    pub k: u32,
    pub out_sum: &'a BufferRef,
    pub workspace: &'a BufferRef,
}

impl KernelCall for MoePrefillCall<'_> {
    fn encode(&self, k: &Kernels) -> Result<(), SmoeError> {
        let s = self.shape.raw();
        check(unsafe {
            sys::smoe_moe_prefill(k.h, &s, self.experts.ptr, self.stride, self.n_experts,
                                  self.indices.ptr as *const i32, self.weights.ptr as *const f32, self.input.ptr,
                                  self.input_is_bf16 as c_int, self.n_tokens, self.k,
                                  self.out_sum.ptr as *mut f32, self.workspace.ptr, self.workspace.len)
        }, "smoe_moe_prefill")
    }
}

/// The whole prefill MoE block of one layer (linear_attn_forward.rs:
/// 3998-4075): the routed experts as [`MoePrefillCall`], an optional 4-bit
/// shared expert over all tokens with an optional f32 gate vector, and the
/// residual: `hidden_out = (h_mid + moe_sum) + sigmoid(gate . x_t) *
/// shared_out` (`Op::MoeCombineResidualNTokens`). Workspace:
/// [`Kernels::moe_prefill_block_workspace_size`] bytes.
pub struct MoePrefillBlockCall<'a> {
    pub routed: MoePrefillCall<'a>,
    pub shared_expert: Option<&'a BufferRef>,
    pub shared_gate: Option<&'a BufferRef>,
    pub h_mid: &'a BufferRef,
}

impl KernelCall for MoePrefillBlockCall<'_> {
    fn encode(&self, k: &Kernels) -> Result<(), SmoeError> {
        let r = &self.routed;
        let s = r.shape.raw();
        check(unsafe {
            sys::smoe_moe_prefill_block(k.h, &s, r.experts.ptr, r.stride, r.n_experts, r.indices.ptr as *const i32,
                                        r.weights.ptr as *const f32, r.input.ptr, r.input_is_bf16 as c_int,
                                        r.n_tokens, r.k,
                                        self.shared_expert.map_or(ptr::null(), |b| b.ptr as *const c_void),
                                        self.shared_gate.map_or(ptr::null(), |b| b.ptr as *const f32),
                                        self.h_mid.ptr as *const f32, r.out_sum.ptr as *mut f32, r.workspace.ptr,
                                        r.workspace.len)
        }, "smoe_moe_prefill_block")
    }
}

/// The router softmax alone (`softmax`, moe_router.rs:52-72), the
/// reference's probabilities bit for bit, per row of `n` logits.
pub struct SoftmaxCall<'a> {
    pub logits: &'a BufferRef,
    pub n_tokens: u32,
    pub n: u32,
    pub probs: &'a BufferRef,
}

impl KernelCall for SoftmaxCall<'_> {
    fn encode(&self, k: &Kernels) -> Result<(), SmoeError> {
        let what = "smoe_softmax";
        let m = self.n_tokens as u64 * self.n as u64;
        let l = self.logits.f32_span(0, m, what)?;
        let p = self.probs.f32_span(0, m, what)?;
        check(unsafe { sys::smoe_softmax(k.h, l, self.n_tokens, self.n, p) }, what)
    }
}

/// Layout and expert stride of a `layer_NN.bin` of `file_bytes` bytes
/// (`layout_and_stride`, io/expert_io.rs:229-267): `(bits, expert_size,
/// stride)`.
pub fn layer_file_layout(file_bytes: u64, n_experts: u32, hidden: u32, inter: u32, group: u32,
                         declared: Option<(u64, u64)>) -> Result<(u32, u64, u64), SmoeError> {
    let (ds, dst) = declared.unwrap_or((0, 0));
    let mut out = sys::smoe_file_layout::default();
    check(unsafe { sys::smoe_layer_file_layout(file_bytes, n_experts, hidden, inter, group, ds, dst, &mut out) },
          "smoe_layer_file_layout")?;
    Ok((out.bits, out.expert_size, out.stride))
}
