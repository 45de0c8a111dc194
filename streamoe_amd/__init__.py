"""streamoe_amd — MI355X (gfx950) routed-expert MoE hot path.

Host-side mirror of the reference's kernel-crate and expert-encoder
interface over the C ABI of ``libsmoe.so`` (``include/smoe.h``). Names
follow the reference:

* ``ExpertLayout``      crates/streammoe/src/riir/variants.rs:401-486
* ``Kernels``           crates/streammoe-metal/src/lib.rs:538-676 (Kernels::new / encode)
* ``QuantWeights``      crates/streammoe-metal/src/lib.rs:339-351
* ``ExpertPayload``     crates/streammoe/src/riir/moe/expert_forward.rs:123-139
* ``gpu_batched_experts_forward``  expert_forward.rs:718-746
* ``moe_router``        crates/streammoe/src/riir/moe/moe_router.rs:151-181 (on the GPU)
* ``ExpertFiles``, ``layout_and_stride``, ``declared_stride``
                        crates/streammoe/src/riir/io/expert_io.rs:229-420 (resident layers)

Device buffers are torch tensors on ``cuda`` (PyTorch is only the
allocator and stream provider here). Every call goes through libsmoe;
nothing falls back to a CPU path: importing this package without the
built library raises ImportError.
"""
import ctypes as C
import json
import os
from dataclasses import dataclass

from . import _abi
from ._abi import SMOE_MAX_K, SmoeError, check

_lib = _abi.load()

MAX_K = SMOE_MAX_K


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


@dataclass(frozen=True)
class ExpertLayout:
    """Packed-expert layout `[gate | up | down]`, each block
    `[codes | bf16 scales | bf16 biases]` (variants.rs:401-486), for any
    shape: `bits` 4 (8 nibbles per u32, low first) or 3 (8 codes per 3
    bytes, little-endian 24-bit pack)."""

    hidden: int
    inter: int
    bits: int = 4
    group: int = 64

    def row_bytes(self, in_dim):
        return in_dim * self.bits // 8

    @property
    def weight_bytes(self):
        return self.inter * self.row_bytes(self.hidden)

    @property
    def scale_bytes(self):
        return self.inter * (self.hidden // self.group) * 2

    @property
    def block_bytes(self):
        return self.weight_bytes + 2 * self.scale_bytes

    @property
    def expert_size(self):
        return 3 * self.block_bytes

    def offsets(self, block):
        """(codes, scales, biases) byte offsets of block 0=gate, 1=up, 2=down."""
        w = block * self.block_bytes
        s = w + self.weight_bytes
        return w, s, s + self.scale_bytes

    @classmethod
    def from_expert_size(cls, size, hidden, inter, group=64):
        """ExpertLayout::from_expert_size: the layout whose expert is `size` bytes."""
        for bits in (4, 3):
            lay = cls(hidden, inter, bits, group)
            if lay.expert_size == size:
                return lay
        return None

    def shape(self):
        return _abi.ExpertShape(self.hidden, self.inter, self.group, self.bits)


@dataclass
class QuantWeights:
    """One quantized [out_dim, in_dim] matrix inside a device tensor."""

    buffer: object  # torch tensor on the device
    packed_offset: int
    scales_offset: int
    biases_offset: int
    group_size: int = 64
    bits: int = 4

    def c(self):
        return _abi.QWeights(self.buffer.data_ptr(), self.packed_offset, self.scales_offset,
                             self.biases_offset, self.group_size, self.bits)


@dataclass
class ExpertPayload:
    """Per-token host inputs of a K-expert dispatch (expert_forward.rs:123-139)."""

    h_post: object
    h_mid: object
    shared_out: object
    expert_weights: object
    shared_gate_score: float


class Kernels:
    """A libsmoe handle on one GPU: Kernels::new plus the MoeBuffers scratch.

    ``stream`` is a torch.cuda.Stream (default: torch's current stream)."""

    def __init__(self, device=0, stream=None):
        import torch

        self._torch = torch
        self.device = device
        h = C.c_void_p()
        s = (stream or torch.cuda.current_stream(device)).cuda_stream
        check(_lib.smoe_create(device, C.c_void_p(s), C.byref(h)), "smoe_create")
        self.h = h

    def close(self):
        if self.h:
            _lib.smoe_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sync(self):
        check(_lib.smoe_sync(self.h), "smoe_sync")

    def set_stream(self, stream):
        """Launch on `stream` (a torch.cuda.Stream) from now on (smoe_set_stream)."""
        check(_lib.smoe_set_stream(self.h, C.c_void_p(stream.cuda_stream)), "smoe_set_stream")

    def set_option(self, option, value):
        check(_lib.smoe_set_option(self.h, option, value), "smoe_set_option")

    def set_decode_path(self, path):
        """0 auto, 1 one kernel per phase, 3 three-kernel only (SMOE_OPT_DECODE_PATH)."""
        self.set_option(_abi.SMOE_OPT_DECODE_PATH, path)

    def set_prefill_gemm(self, path):
        """0 auto (32 x 32 gate/up and down tiles where they apply), 1 k_pf_mm only, 2 as 0 with the down
        GEMM on k_pf_mm (SMOE_OPT_PREFILL_GEMM)."""
        self.set_option(_abi.SMOE_OPT_PREFILL_GEMM, path)

    def reserve(self, max_hidden, max_inter, max_experts):
        check(_lib.smoe_reserve(self.h, max_hidden, max_inter, max_experts), "smoe_reserve")

    # -- dense quantized matvec (encode_matvec / QmmCall with one token) ----------
    def qmv(self, w: QuantWeights, x, y, out_dim, in_dim):
        wc = w.c()
        return _lib.smoe_qmv(self.h, C.byref(wc), _ptr(x), _ptr(y), out_dim, in_dim)

    def qmv_argmax(self, w: QuantWeights, x, y, out_dim, in_dim, out):
        """qmv with the argmax of y fused (LM head + greedy pick)."""
        wc = w.c()
        return _lib.smoe_qmv_argmax(self.h, C.byref(wc), _ptr(x), _ptr(y), out_dim, in_dim, _ptr(out))

    def qmm_workspace_size(self, in_dim, group, n_tokens):
        return _lib.smoe_qmm_workspace_size(in_dim, group, n_tokens)

    def qmm(self, w: QuantWeights, x, y, out_dim, in_dim, n_tokens, workspace):
        """QmmCall (metal/lib.rs:357-380): y[n, out] = x[n, in] . dequant(W)^T."""
        wc = w.c()
        return _lib.smoe_qmm(self.h, C.byref(wc), _ptr(x), _ptr(y), out_dim, in_dim, n_tokens,
                             _ptr(workspace), workspace.numel() * workspace.element_size())

    def argmax(self, v, n, out):
        return _lib.smoe_argmax(self.h, _ptr(v), n, _ptr(out))

    def dequant(self, w: QuantWeights, in_dim, row0, n_rows, out):
        wc = w.c()
        return _lib.smoe_dequant(self.h, C.byref(wc), in_dim, row0, n_rows, _ptr(out))

    # -- router ------------------------------------------------------------------
    def router(self, router_w, x, n_tokens, n_experts, hidden, k, normalize, idx, weights,
               logits=None):
        return _lib.smoe_router(self.h, _ptr(router_w), _ptr(x), n_tokens, n_experts, hidden, k,
                                int(normalize), _ptr(idx), _ptr(weights), _ptr(logits))

    def softmax_topk(self, logits, n_tokens, n_experts, k, normalize, idx, weights):
        return _lib.smoe_softmax_topk(self.h, _ptr(logits), n_tokens, n_experts, k, int(normalize),
                                      _ptr(idx), _ptr(weights))

    def softmax(self, logits, n_tokens, n, probs):
        """softmax() of moe_router.rs:52-72 per row, the reference's bits."""
        return _lib.smoe_softmax(self.h, _ptr(logits), n_tokens, n, _ptr(probs))

    def expf(self, x, y, n):
        """glibc's expf (the reference softmax's exponential) on the device."""
        return _lib.smoe_expf(self.h, _ptr(x), _ptr(y), n)

    def topk(self, scores, n_tokens, n, k, idx, values):
        return _lib.smoe_topk(self.h, _ptr(scores), n_tokens, n, k, _ptr(idx), _ptr(values))

    def noaux_tc_topk(self, logits, correction_bias, n_tokens, n_experts, n_group, topk_group, k,
                      routed_scaling_factor, idx, weights, scores_out=None):
        """noaux_tc_router_cpu (moe_router.rs:211-330) on the device."""
        return _lib.smoe_noaux_tc_topk(self.h, _ptr(logits), _ptr(correction_bias), n_tokens, n_experts,
                                       n_group, topk_group, k, float(routed_scaling_factor), _ptr(idx),
                                       _ptr(weights), _ptr(scores_out))

    # -- decode experts (encode_experts_mmap_into) --------------------------------
    def experts_decode(self, layout: ExpertLayout, bindings, weights, input, h_mid, shared_out,
                       shared_gate_score, hidden_out):
        """bindings: list of (tensor, byte_offset); weights: list of floats."""
        k = len(bindings)
        b = (_abi.Binding * max(k, 1))(*[_abi.Binding(t.data_ptr(), off) for t, off in bindings])
        w = (C.c_float * max(k, 1))(*weights)
        shape = layout.shape()
        return _lib.smoe_experts_decode(self.h, C.byref(shape), b, k, w, _ptr(input), _ptr(h_mid),
                                        _ptr(shared_out), C.c_float(shared_gate_score),
                                        _ptr(hidden_out))

    # -- one resident layer (moe_dispatch_per_token with device routing) --------
    @staticmethod
    def layer(layout: ExpertLayout, experts, stride, n_experts, k, normalize, router_w,
              shared_expert=None, shared_gate=None, router_q=None, shared_gate_q=None):
        """router_w: f32 router tensor, or None with router_q (an 8-bit
        QuantWeights [n_experts, hidden]); shared_gate_q: an 8-bit shared gate
        [1, hidden] in place of shared_gate."""
        rq = None if router_q is None else router_q.c()
        gq = None if shared_gate_q is None else shared_gate_q.c()
        L = _abi.Layer(layout.shape(), experts.data_ptr(), stride, n_experts, k, int(normalize),
                       None if router_w is None else router_w.data_ptr(),
                       None if shared_expert is None else shared_expert.data_ptr(),
                       None if shared_gate is None else shared_gate.data_ptr(),
                       None if rq is None else C.addressof(rq), None if gq is None else C.addressof(gq))
        L._keep = (rq, gq)  # the smoe_qweights structs the layer points to
        return L

    def moe_decode_layer(self, layer, input, h_mid, hidden_out, idx_out=None, w_out=None):
        return _lib.smoe_moe_decode_layer(self.h, C.byref(layer), _ptr(input), _ptr(h_mid),
                                          _ptr(hidden_out), _ptr(idx_out), _ptr(w_out))

    def moe_decode_layers(self, layers, norm_w, eps, input, residual_io, work):
        n = len(layers)
        arr = (_abi.Layer * n)(*layers)
        nw = None
        if norm_w is not None:
            nw = (C.c_void_p * n)(*[None if t is None else t.data_ptr() for t in norm_w])
        return _lib.smoe_moe_decode_layers(self.h, arr, n, nw, C.c_float(eps), _ptr(input),
                                           _ptr(residual_io), _ptr(work))

    def moe_decode_tokens(self, layers, norm_w, eps, n_tokens, input, residual_io, work, idx_out=None,
                          w_out=None):
        """T <= 4 tokens through the layers at once (decode_multi.rs
        moe_dispatch_multi); rows of input / residual_io / work are tokens."""
        n = len(layers)
        arr = (_abi.Layer * n)(*layers)
        nw = None
        if norm_w is not None:
            nw = (C.c_void_p * n)(*[None if t is None else t.data_ptr() for t in norm_w])
        return _lib.smoe_moe_decode_tokens(self.h, arr, n, nw, C.c_float(eps), n_tokens, _ptr(input),
                                           _ptr(residual_io), _ptr(work), _ptr(idx_out), _ptr(w_out))

    # -- prefill (encode_moe_gather_id_fuse) --------------------------------------
    def moe_prefill_workspace_size(self, layout, n_tokens, n_experts, k):
        shape = layout.shape()
        return _lib.smoe_moe_prefill_workspace_size(C.byref(shape), n_tokens, n_experts, k)

    def moe_prefill(self, layout, experts, stride, n_experts, idx, weights, x, x_is_bf16, n_tokens,
                    k, out_sum, workspace):
        shape = layout.shape()
        return _lib.smoe_moe_prefill(self.h, C.byref(shape), _ptr(experts), stride, n_experts,
                                     _ptr(idx), _ptr(weights), _ptr(x), int(x_is_bf16), n_tokens, k,
                                     _ptr(out_sum), _ptr(workspace),
                                     0 if workspace is None else workspace.numel() * workspace.element_size())

    def moe_prefill_block_workspace_size(self, layout, n_tokens, n_experts, k, has_shared):
        shape = layout.shape()
        return _lib.smoe_moe_prefill_block_workspace_size(C.byref(shape), n_tokens, n_experts, k, int(has_shared))

    def moe_prefill_block(self, layout, experts, stride, n_experts, idx, weights, x, x_is_bf16, n_tokens, k,
                          shared, gate, h_mid, hidden_out, workspace):
        """The prefill MoE block (linear_attn_forward.rs:3998-4075): routed
        experts, optional shared expert with sigmoid gate, residual."""
        shape = layout.shape()
        return _lib.smoe_moe_prefill_block(self.h, C.byref(shape), _ptr(experts), stride, n_experts, _ptr(idx),
                                           _ptr(weights), _ptr(x), int(x_is_bf16), n_tokens, k, _ptr(shared),
                                           _ptr(gate), _ptr(h_mid), _ptr(hidden_out), _ptr(workspace),
                                           0 if workspace is None else workspace.numel() * workspace.element_size())

    # -- expert files -------------------------------------------------------------
    def load_file(self, path, dst, offset=0, nbytes=0):
        """Copy bytes [offset, offset + nbytes) of the file (nbytes 0: to its
        end) into the device tensor dst; returns the bytes copied."""
        got = C.c_uint64(0)
        check(_lib.smoe_load_file(self.h, os.fsencode(path), offset, nbytes, _ptr(dst),
                                  dst.numel() * dst.element_size(), C.byref(got)), f"smoe_load_file({path})")
        return got.value

    # -- diagnostics --------------------------------------------------------------
    def stream_read(self, buf, nbytes, sink):
        """Read nbytes of the device tensor `buf` once (HBM read-peak probe)."""
        return _lib.smoe_stream_read(self.h, _ptr(buf), nbytes, _ptr(sink))

    # -- synthetic data ---------------------------------------------------------
    def synth_experts(self, base, n_experts, stride, layout, seed, scale_sigma=0.02,
                      bias_sigma=0.01):
        shape = layout.shape()
        return _lib.smoe_synth_experts(self.h, _ptr(base), n_experts, stride, C.byref(shape), seed,
                                       C.c_float(scale_sigma), C.c_float(bias_sigma))

    def synth_normal_f32(self, out, seed, sigma=1.0):
        return _lib.smoe_synth_normal_f32(self.h, _ptr(out), out.numel(), seed, C.c_float(sigma))

    def synth_normal_bf16(self, out, seed, sigma=1.0):
        return _lib.smoe_synth_normal_bf16(self.h, _ptr(out), out.numel(), seed, C.c_float(sigma))


class ExpertIoError(RuntimeError):
    """ExpertIoError (io/expert_io.rs): Io, MixedLayouts."""


def declared_stride(packed_dir):
    """declared_stride (expert_io.rs:239-251): (expert_size, expert_stride)
    from packed_dir/layout.json when it declares a stride above the size,
    else None."""
    try:
        with open(os.path.join(packed_dir, "layout.json")) as f:
            v = json.load(f)
        size, stride = int(v["expert_size"]), int(v["expert_stride"])
    except (OSError, ValueError, KeyError, TypeError):
        return None
    return (size, stride) if stride > size else None


def layout_and_stride(file_bytes, n_experts, hidden, inter, group=64, declared=None):
    """layout_and_stride (expert_io.rs:253-267) through libsmoe: the
    (ExpertLayout, stride) of a layer file file_bytes long."""
    out = _abi.FileLayout()
    ds, dst = declared if declared else (0, 0)
    check(_lib.smoe_layer_file_layout(file_bytes, n_experts, hidden, inter, group, ds, dst, C.byref(out)),
          "smoe_layer_file_layout")
    return ExpertLayout(hidden, inter, out.bits, group), out.stride


class ExpertFiles:
    """Resident expert arenas from experts_dir/packed_experts/layer_NN.bin
    (ExpertFiles::open_range_tiered, expert_io.rs:332-420, with every layer
    loaded into one device arena: expert e of layer l at arena(l) + e *
    stride). Missing layer files stay None; layers whose layouts differ
    raise ExpertIoError (MixedLayouts); a layout.json padded stride is
    honoured as the reference does."""

    def __init__(self, kernels: Kernels, experts_dir, n_layers, n_experts, hidden, inter, group=64,
                 layers=None):
        import torch

        packed = os.path.join(experts_dir, "packed_experts")
        declared = declared_stride(packed)
        self.layout = None
        self.stride = None
        self.arenas = [None] * n_layers
        first = None
        for i in (range(n_layers) if layers is None else layers):
            path = os.path.join(packed, f"layer_{i:02d}.bin")
            try:
                size = os.path.getsize(path)
            except FileNotFoundError:
                continue
            lay, stride = layout_and_stride(size, n_experts, hidden, inter, group, declared)
            if first is None:
                first = i
                self.layout, self.stride = lay, stride
            elif lay.bits != self.layout.bits:
                raise ExpertIoError(f"MixedLayouts: layer {i} is {lay.bits}-bit, layer {first} is "
                                    f"{self.layout.bits}-bit")
            arena = torch.empty(size, dtype=torch.uint8, device=f"cuda:{kernels.device}")
            kernels.load_file(path, arena)
            self.arenas[i] = arena
        if self.layout is None:
            self.layout, self.stride = ExpertLayout(hidden, inter, 4, group), None

    def arena(self, layer):
        return self.arenas[layer]

    def binding(self, layer, expert):
        """(arena, byte offset) of one expert: the reference's (&Buffer, u64)."""
        return self.arenas[layer], expert * self.stride


def zipf_routing(n_tokens, n_experts, k, s=1.1, seed=0):
    """Synthetic prefill routing (the skewed config-4 workload): per token,
    k distinct experts drawn by Gumbel-top-k with p_e proportional to
    rank_e^-s over a seeded permutation of the experts; weights = softmax of
    k seeded N(0, 1) logits. Returns (idx int32 [n, k], w float32 [n, k])."""
    import numpy as np

    rng = np.random.default_rng(seed)
    ranks = np.empty(n_experts)
    ranks[rng.permutation(n_experts)] = np.arange(1, n_experts + 1)
    logp = -s * np.log(ranks)
    keys = logp[None, :] + rng.gumbel(size=(n_tokens, n_experts))
    idx = np.argsort(-keys, axis=1, kind="stable")[:, :k].astype(np.int32)
    lg = rng.standard_normal((n_tokens, k))
    w = np.exp(lg - lg.max(axis=1, keepdims=True))
    w /= w.sum(axis=1, keepdims=True)
    return idx, w.astype(np.float32)


def capture_graph(kernels: Kernels, fn):
    """Record the launches `fn()` makes on `kernels` into a HIP graph (torch's
    CUDAGraph over hipGraph) and return it; fn runs once eagerly on the
    capture stream first. The handle launches on torch's current stream
    again afterwards. Only launch sequences that allocate nothing and set no
    memory (the per-phase and three-kernel decode) can be captured."""
    import torch

    dev = torch.device("cuda", kernels.device)
    stream = torch.cuda.current_stream(dev)
    side = torch.cuda.Stream(dev)
    side.wait_stream(stream)
    try:
        with torch.cuda.stream(side):
            kernels.set_stream(side)
            fn()
        stream.wait_stream(side)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            kernels.set_stream(torch.cuda.current_stream(dev))
            fn()
    finally:
        kernels.set_stream(stream)
    torch.cuda.synchronize(dev)
    return graph


def gpu_batched_experts_forward(kernels: Kernels, layout: ExpertLayout, actual_k, expert_data,
                                payload: ExpertPayload):
    """K expert blobs (host bytes, slot order) through gate/up/SwiGLU/down and
    the combine; returns the post-combine hidden state (host float32).
    Mirrors expert_forward.rs:718-746 (stage, dispatch, wait, read back)."""
    import numpy as np
    import torch

    if actual_k < 1 or actual_k > MAX_K:
        raise SmoeError(_abi.CODES["SMOE_ERR_BAD_K"], "gpu_batched_experts_forward")
    data = np.frombuffer(bytes(expert_data), np.uint8).copy()  # writable, for torch.from_numpy
    if data.size != actual_k * layout.expert_size:
        raise SmoeError(_abi.CODES["SMOE_ERR_INVALID_ARG"], "expert_data length")
    dev = torch.device("cuda", kernels.device)
    blobs = torch.from_numpy(data).to(dev)
    f = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)
    x, h_mid, shared = f(payload.h_post), f(payload.h_mid), f(payload.shared_out)
    out = torch.empty(layout.hidden, dtype=torch.float32, device=dev)
    bindings = [(blobs, s * layout.expert_size) for s in range(actual_k)]
    check(kernels.experts_decode(layout, bindings, list(payload.expert_weights), x, h_mid, shared,
                                 payload.shared_gate_score, out), "smoe_experts_decode")
    kernels.sync()
    return out.cpu().numpy()
