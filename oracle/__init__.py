"""Python view of the CPU oracle (liboracle.so, built from oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product (streamoe_amd/).
Every function is a numpy-in / numpy-out wrapper of the C restatement of
the reference's CPU path; see oracle.h for the reference citations.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build():
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_P = C.c_void_p
_U32 = C.c_uint32


def _declare(L):
    sig = {
        "orc_bf16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "orc_expert_bytes": (C.c_size_t, [_U32, _U32, _U32, _U32]),
        "orc_expert_offsets": (None, [_U32, _U32, _U32, _U32, _U32, _P]),
        "orc_dequant_4bit": (None, [_P, _P, _P, _U32, _U32, _U32, _P]),
        "orc_dequant_8bit": (None, [_P, _P, _P, _U32, _U32, _U32, _P]),
        "orc_dequant_matvec_4bit_gs": (C.c_int, [_P, _P, _P, _U32, _U32, _U32, _P, _P, C.c_int]),
        "orc_dequant_matvec_8bit_gs": (C.c_int, [_P, _P, _P, _U32, _U32, _U32, _P, _P, C.c_int]),
        "orc_lm_head": (C.c_int, [_P, _P, _P, _U32, _U32, _U32, _P, _P]),
        "orc_f32_matvec": (None, [_P, _U32, _U32, _P, _P]),
        "orc_argmax": (_U32, [_P, _U32]),
        "orc_pack_3bit": (None, [_P, C.c_size_t, _P]),
        "orc_q3_expert_to_q4": (C.c_int, [_P, _U32, _U32, _U32, _P]),
        "orc_expert_swiglu": (C.c_int, [_P, _U32, _U32, _U32, _U32, _P, _P, C.c_int]),
        "orc_softmax": (C.c_int, [_P, _U32]),
        "orc_softmax_rows": (C.c_int, [_P, _U32, _U32, C.c_int]),
        "orc_moe_combine_residual_n_tokens": (None, [_P, _P, _P, _P, _P, _U32, _U32]),
        "orc_expf_many": (C.c_int, [_P, _P, C.c_uint64, C.c_int]),
        "orc_topk": (C.c_int, [_P, _U32, _U32, _P, _P]),
        "orc_normalize_weights": (None, [_P, _U32]),
        "orc_router": (C.c_int, [_P, _U32, _U32, C.c_int, _P, _P]),
        "orc_sigmoid": (C.c_float, [C.c_float]),
        "orc_noaux_tc_router": (C.c_int, [_P, _P, _U32, _U32, _U32, _U32, C.c_float, _P, _P]),
        "orc_combine": (None, [_P, _P, _U32, _P, _P, C.c_float, _U32, _P]),
        "orc_moe_decode_layer": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, C.c_int]),
        "orc_rms_norm_bf16": (None, [_P, _P, _U32, C.c_float, _P]),
        "orc_build_expert_buckets": (C.c_int, [_P, _P, _U32, _U32, _U32, _P, _P, _P, _P, _P]),
        "orc_xorshift64s": (C.c_uint64, [C.c_uint64, _P, C.c_size_t]),
        "orc_moe_permute_fuse": (C.c_int, [_P, C.c_uint64, _U32, _U32, _U32, _U32, _P, _P, _P, _U32,
                                           _P, _P, _P, C.c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _words(a):
    """Packed 4-bit codes as little-endian u32 words; a byte array is
    reinterpreted (not converted element by element)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint8:
        return a.view(np.uint32)
    return _c(a, np.uint32)


class OrcLayer(C.Structure):
    _fields_ = [
        ("hidden", _U32), ("inter", _U32), ("n_experts", _U32), ("k", _U32), ("group", _U32),
        ("bits", _U32), ("normalize", C.c_int), ("experts", _P), ("stride", C.c_uint64),
        ("router_w", _P), ("shared_blob", _P), ("shared_inter", _U32), ("shared_gate_w", _P),
        ("router_q8", _P), ("router_s8", _P), ("router_b8", _P), ("gate_q8", _P), ("gate_s8", _P),
        ("gate_b8", _P), ("group8", _U32),
    ]


# ---- bf16 / layout ---------------------------------------------------------
def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x):
    """Round to nearest even as the reference's generators
    (crates/streammoe/tests/matvec_decode_bench.rs:36-39)."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + (((b >> 16) & 1) + 0x7FFF)) >> 16).astype(np.uint16)


def expert_bytes(hidden, inter, bits, group):
    return lib().orc_expert_bytes(hidden, inter, bits, group)


def expert_offsets(hidden, inter, bits, group, block):
    out = np.zeros(3, np.uint64)
    lib().orc_expert_offsets(hidden, inter, bits, group, block, _p(out))
    return tuple(int(v) for v in out)


# ---- dequant / matvec ------------------------------------------------------
def dequant_4bit(packed, scales, biases, in_dim, out_dim, group):
    packed, scales, biases = _words(packed), _c(scales, np.uint16), _c(biases, np.uint16)
    out = np.empty((out_dim, in_dim), np.float32)
    lib().orc_dequant_4bit(_p(packed), _p(scales), _p(biases), in_dim, out_dim, group, _p(out))
    return out


def dequant_8bit(packed, scales, biases, in_dim, out_dim, group):
    """packed: bytes [out_dim, in_dim] (or their u32 words)."""
    packed, scales, biases = _words(packed), _c(scales, np.uint16), _c(biases, np.uint16)
    out = np.empty((out_dim, in_dim), np.float32)
    lib().orc_dequant_8bit(_p(packed), _p(scales), _p(biases), in_dim, out_dim, group, _p(out))
    return out


def dequant_matvec_4bit_gs(packed, scales, biases, in_dim, out_dim, group, x, nthreads=0):
    packed, scales, biases = _words(packed), _c(scales, np.uint16), _c(biases, np.uint16)
    x = _c(x, np.float32)
    out = np.empty(out_dim, np.float32)
    rc = lib().orc_dequant_matvec_4bit_gs(_p(packed), _p(scales), _p(biases), in_dim, out_dim,
                                          group, _p(x), _p(out), nthreads)
    return rc, out


def dequant_matvec_8bit_gs(packed, scales, biases, in_dim, out_dim, group, x, nthreads=0):
    """packed: bytes [out_dim, in_dim] (or their u32 words, byte n of word i =
    input 4i + n); scales / biases: bf16 [out_dim, in_dim / group]."""
    packed, scales, biases = _words(packed), _c(scales, np.uint16), _c(biases, np.uint16)
    x = _c(x, np.float32)
    out = np.empty(out_dim, np.float32)
    rc = lib().orc_dequant_matvec_8bit_gs(_p(packed), _p(scales), _p(biases), in_dim, out_dim,
                                          group, _p(x), _p(out), nthreads)
    return rc, out


def lm_head(packed, scales, biases, hidden, vocab, group, x):
    packed, scales, biases = _words(packed), _c(scales, np.uint16), _c(biases, np.uint16)
    x = _c(x, np.float32)
    out = np.empty(vocab, np.float32)
    rc = lib().orc_lm_head(_p(packed), _p(scales), _p(biases), hidden, vocab, group, _p(x), _p(out))
    assert rc == 0
    return out


def f32_matvec(w, x):
    w, x = _c(w, np.float32), _c(x, np.float32)
    out = np.empty(w.shape[0], np.float32)
    lib().orc_f32_matvec(_p(w), w.shape[1], w.shape[0], _p(x), _p(out))
    return out


def argmax(v):
    v = _c(v, np.float32)
    return int(lib().orc_argmax(_p(v), v.size))


# ---- 3-bit ------------------------------------------------------------------
def pack_3bit(words4):
    words4 = _words(words4).ravel()
    out = np.empty(words4.size * 3, np.uint8)
    lib().orc_pack_3bit(_p(words4), words4.size, _p(out))
    return out


def q3_expert_to_q4(blob3, hidden, inter, group):
    blob3 = _c(blob3, np.uint8)
    out = np.empty(expert_bytes(hidden, inter, 4, group), np.uint8)
    assert lib().orc_q3_expert_to_q4(_p(blob3), hidden, inter, group, _p(out)) == 0
    return out


# ---- expert FFN ---------------------------------------------------------------
def expert_swiglu(blob, bits, hidden, inter, group, x, nthreads=0):
    blob, x = _c(blob, np.uint8), _c(x, np.float32)
    out = np.empty(hidden, np.float32)
    rc = lib().orc_expert_swiglu(_p(blob), bits, hidden, inter, group, _p(x), _p(out), nthreads)
    assert rc == 0, rc
    return out


# ---- router -------------------------------------------------------------------
def softmax(x):
    x = np.array(x, np.float32)
    assert lib().orc_softmax(_p(x), x.size) == 0
    return x


def softmax_rows(x, nthreads=0):
    """orc_softmax on every row of a 2-D float32 array (rows in parallel)."""
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    assert lib().orc_softmax_rows(_p(x), x.shape[0], x.shape[1], nthreads) == 0
    return x


def expf_many(x, nthreads=0):
    """The host libm's expf on every element (the reference softmax's exp)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    assert lib().orc_expf_many(_p(x), _p(y), x.size, nthreads) == 0
    return y


def topk(scores, k):
    scores = _c(scores, np.float32)
    idx, val = np.empty(k, np.int32), np.empty(k, np.float32)
    rc = lib().orc_topk(_p(scores), scores.size, k, _p(idx), _p(val))
    return rc, idx, val


def normalize_weights(w):
    w = np.array(w, np.float32)
    lib().orc_normalize_weights(_p(w), w.size)
    return w


def router(scores, k, normalize):
    s = np.array(scores, np.float32)
    idx, w = np.empty(k, np.int32), np.empty(k, np.float32)
    rc = lib().orc_router(_p(s), s.size, k, int(normalize), _p(idx), _p(w))
    return rc, idx, w


def sigmoid(x):
    return lib().orc_sigmoid(float(x))


def noaux_tc_router(logits, bias, n_group, topk_group, k, scale):
    """noaux_tc_router_cpu (moe_router.rs:211-330); returns (rc, idx, w,
    scores) with scores = sigmoid(logits), as the reference leaves them."""
    s = np.array(logits, np.float32)
    b = _c(bias, np.float32)
    idx, w = np.empty(k, np.int32), np.empty(k, np.float32)
    rc = lib().orc_noaux_tc_router(_p(s), _p(b), s.size, n_group, topk_group, k, float(scale), _p(idx), _p(w))
    return rc, idx, w, s


def combine(expert_out, weights, h_mid, shared_out=None, shared_gate_score=float("nan")):
    expert_out, weights, h_mid = _c(expert_out, np.float32), _c(weights, np.float32), _c(h_mid, np.float32)
    so = None if shared_out is None else _c(shared_out, np.float32)
    out = np.empty(h_mid.size, np.float32)
    lib().orc_combine(_p(expert_out), _p(weights), weights.size, _p(h_mid), _p(so),
                      float(shared_gate_score), h_mid.size, _p(out))
    return out


def moe_decode_layer(experts, stride, hidden, inter, n_experts, k, group, bits, normalize, router_w,
                     x, h_mid, shared_blob=None, shared_gate_w=None, nthreads=0, router_q8=None,
                     gate_q8=None):
    """One decode layer on the CPU; returns (hidden_out, idx, w, logits).
    router_q8 / gate_q8: an 8-bit affine router [n_experts, hidden] / shared
    gate [1, hidden] as (codes uint8, scales bf16, biases bf16, group),
    used instead of router_w / shared_gate_w."""
    experts = _c(experts, np.uint8)
    x, h_mid = _c(x, np.float32), _c(h_mid, np.float32)
    router_w = None if router_w is None else _c(router_w, np.float32)
    sb = None if shared_blob is None else _c(shared_blob, np.uint8)
    sg = None if shared_gate_w is None else _c(shared_gate_w, np.float32)
    keep = []

    def q8(t):
        if t is None:
            return None, None, None, 0
        q, s, b, g = _c(t[0], np.uint8), _c(t[1], np.uint16), _c(t[2], np.uint16), int(t[3])
        keep.extend((q, s, b))
        return q.ctypes.data, s.ctypes.data, b.ctypes.data, g
    rq, rs, rb, rg = q8(router_q8)
    gq, gs_, gb, gg = q8(gate_q8)
    assert router_w is not None or rq is not None
    assert not (rg and gg) or rg == gg
    L = OrcLayer(hidden, inter, n_experts, k, group, bits, int(normalize), experts.ctypes.data,
                 stride, None if router_w is None else router_w.ctypes.data,
                 None if sb is None else sb.ctypes.data, inter, None if sg is None else sg.ctypes.data,
                 rq, rs, rb, gq, gs_, gb, rg or gg)
    out = np.empty(hidden, np.float32)
    idx, w = np.empty(k, np.int32), np.empty(k, np.float32)
    logits = np.empty(n_experts, np.float32)
    rc = lib().orc_moe_decode_layer(C.byref(L), _p(x), _p(h_mid), _p(out), _p(idx), _p(w),
                                    _p(logits), nthreads)
    assert rc == 0, rc
    return out, idx, w, logits


def rms_norm_bf16(x, w_bf16, eps):
    x, w = _c(x, np.float32), _c(w_bf16, np.uint16)
    out = np.empty(x.size, np.float32)
    lib().orc_rms_norm_bf16(_p(x), _p(w), x.size, C.c_float(eps), _p(out))
    return out


# ---- prefill --------------------------------------------------------------------
def build_expert_buckets(idx, w, n_tokens, k, n_experts):
    idx, w = _c(idx, np.int32).ravel(), _c(w, np.float32).ravel()
    total = n_tokens * k
    eids = np.empty(max(n_experts, 1), np.int32)
    offs = np.empty(max(n_experts, 1) + 1, np.uint32)
    tok = np.empty(max(total, 1), np.int32)
    ws = np.empty(max(total, 1), np.float32)
    nb = np.zeros(1, np.uint32)
    rc = lib().orc_build_expert_buckets(_p(idx), _p(w), n_tokens, k, n_experts, _p(eids), _p(offs),
                                        _p(tok), _p(ws), _p(nb))
    n = int(nb[0])
    return rc, eids[:n].copy(), offs[:n + 1].copy(), tok[:total].copy(), ws[:total].copy()


def moe_permute_fuse(experts, stride, bits, hidden, inter, group, x, buckets, n_tokens,
                     nthreads=0):
    """out_sum[n_tokens, hidden] (zero-initialised) from CSR buckets."""
    _, eids, offs, tok, ws = buckets
    experts, x = _c(experts, np.uint8), _c(x, np.float32)
    eids, offs, tok, ws = _c(eids, np.int32), _c(offs, np.uint32), _c(tok, np.int32), _c(ws, np.float32)
    out = np.zeros((n_tokens, hidden), np.float32)
    rc = lib().orc_moe_permute_fuse(_p(experts), stride, bits, hidden, inter, group, _p(x), _p(eids),
                                    _p(offs), eids.size, _p(tok), _p(ws), _p(out), nthreads)
    assert rc == 0, rc
    return out


def moe_combine_residual_n_tokens(h_mid, moe_sum, shared_out=None, shared_gate=None):
    """hidden = (h_mid + moe_sum) + sigmoid(gate[t]) * shared_out per token
    (backend/cpu/mod.rs:657-695)."""
    h_mid, moe_sum = _c(h_mid, np.float32), _c(moe_sum, np.float32)
    n, dim = h_mid.shape
    so = None if shared_out is None else _c(shared_out, np.float32)
    sg = None if shared_gate is None else _c(shared_gate, np.float32)
    out = np.empty_like(h_mid)
    lib().orc_moe_combine_residual_n_tokens(_p(h_mid), _p(moe_sum), _p(so), _p(sg), _p(out), n, dim)
    return out


def moe_prefill_block(experts, stride, bits, hidden, inter, group, n_experts, x, idx, w, h_mid,
                      shared=None, gate=None, nthreads=0):
    """The prefill MoE block (linear_attn_forward.rs:3998-4075) on the CPU:
    moe_permute_fuse over the routed experts; the shared expert's FFN per
    token (run_packed_expert_swiglu, 4-bit); its gate score gate . x_t (an
    f32 matvec, sequential FMA); moe_combine_residual_n_tokens."""
    x = _c(x, np.float32)
    n, k = idx.shape
    rc, *b = build_expert_buckets(idx, w, n, k, n_experts)
    assert rc == 0, rc
    moe = moe_permute_fuse(experts, stride, bits, hidden, inter, group, x, (rc, *b), n, nthreads)
    so = sg = None
    if shared is not None:
        so = np.stack([expert_swiglu(shared, 4, hidden, inter, group, x[t], nthreads) for t in range(n)])
        if gate is not None:
            sg = np.array([f32_matvec(np.asarray(gate, np.float32)[None, :], x[t])[0] for t in range(n)],
                          np.float32)
    return moe_combine_residual_n_tokens(h_mid, moe, so, sg), moe, so, sg


# ---- test-input generator ---------------------------------------------------------
class XorShift64s:
    """The reference tests' xorshift64* stream (packed_3bit.rs:21-31)."""

    def __init__(self, seed):
        self.state = seed & 0xFFFFFFFFFFFFFFFF

    def next_u64(self, n):
        out = np.empty(n, np.uint64)
        self.state = int(lib().orc_xorshift64s(self.state, _p(out), n))
        return out

    def unit(self, n):
        """packed_3bit.rs unit(): (next >> 40) / 2^24 * 2 - 1, in f32."""
        u = (self.next_u64(n) >> np.uint64(40)).astype(np.float32)
        return (u / np.float32(1 << 24) * np.float32(2.0) - np.float32(1.0)).astype(np.float32)
