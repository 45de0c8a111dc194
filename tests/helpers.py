"""Seeded test-input generators shared by the CPU and GPU tests."""
import numpy as np

import oracle


def bf16(x):
    return oracle.f32_to_bf16(np.asarray(x, np.float32))


def gen_quant_matrix(rng, out_dim, in_dim, group=64, bits=4, ssig=0.02, bsig=0.01):
    """One quantized [out_dim, in_dim] matrix with the BASELINE
    distributions: codes uniform, scales bf16(|N(0, ssig)|), biases
    bf16(N(0, bsig)). Returns (codes bytes, scales u16, biases u16)."""
    n_groups = in_dim // group
    if bits == 4:
        codes = rng.integers(0, 2**32, size=(out_dim, in_dim // 8), dtype=np.uint64).astype(np.uint32)
        codes = codes.view(np.uint8).reshape(out_dim, in_dim // 2)
    elif bits == 8:
        codes = rng.integers(0, 256, size=(out_dim, in_dim), dtype=np.uint8)
    else:
        codes = rng.integers(0, 256, size=(out_dim, in_dim * 3 // 8), dtype=np.uint8)
    scales = bf16(np.abs(rng.standard_normal((out_dim, n_groups))) * ssig)
    biases = bf16(rng.standard_normal((out_dim, n_groups)) * bsig)
    return codes, scales, biases


def gen_expert_blob(rng, hidden, inter, group=64, bits=4):
    """One packed expert [gate | up | down] as uint8 bytes."""
    parts = []
    for blk in range(3):
        out_dim, in_dim = (inter, hidden) if blk < 2 else (hidden, inter)
        c, s, b = gen_quant_matrix(rng, out_dim, in_dim, group, bits)
        parts += [c.ravel(), s.view(np.uint8).ravel(), b.view(np.uint8).ravel()]
    blob = np.concatenate(parts)
    assert blob.size == oracle.expert_bytes(hidden, inter, bits, group)
    return blob


def q4_block_views(blob, hidden, inter, group, block):
    """(packed u32, scales u16, biases u16, in_dim, out_dim) of a 4-bit blob block."""
    w, s, b = oracle.expert_offsets(hidden, inter, 4, group, block)
    out_dim, in_dim = (inter, hidden) if block < 2 else (hidden, inter)
    n = out_dim * in_dim
    packed = blob[w:w + n // 2].view(np.uint32)
    scales = blob[s:s + out_dim * (in_dim // group) * 2].view(np.uint16)
    biases = blob[b:b + out_dim * (in_dim // group) * 2].view(np.uint16)
    return packed, scales, biases, in_dim, out_dim


def dequant_f64(packed_u32, scales, biases, in_dim, out_dim, group):
    """Dequantized matrix in float64 (independent brute force)."""
    words = np.asarray(packed_u32, np.uint32).reshape(out_dim, in_dim // 8).astype(np.uint64)
    shifts = (np.arange(8, dtype=np.uint64) * 4)
    q = ((words[:, :, None] >> shifts) & 0xF).reshape(out_dim, in_dim).astype(np.float64)
    s = oracle.bf16_to_f32(scales).astype(np.float64).reshape(out_dim, -1)
    b = oracle.bf16_to_f32(biases).astype(np.float64).reshape(out_dim, -1)
    s = np.repeat(s, group, axis=1)
    b = np.repeat(b, group, axis=1)
    return q * s + b


def expert_f64(blob4, hidden, inter, group, x):
    """Expert SwiGLU FFN in float64 on a 4-bit blob (independent brute force)."""
    mats = [dequant_f64(*q4_block_views(blob4, hidden, inter, group, b)[:3],
                        *q4_block_views(blob4, hidden, inter, group, b)[3:], group) for b in range(3)]
    x = np.asarray(x, np.float64)
    g, u = mats[0] @ x, mats[1] @ x
    act = g / (1.0 + np.exp(-g)) * u
    return mats[2] @ act


def rel_err(got, want, floor=1e-30):
    """The reference's metric: max|got - want| / max(max|want|, floor)
    (crates/streammoe/tests/group32_kernels.rs:141-150)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(float(np.max(np.abs(want))), floor))


def expert_pair(rng):
    """packed_3bit.rs:34-63 expert_pair at A3B shapes: the same random 3-bit
    codes as 4-bit nibbles and packed 3-bit. rng: oracle.XorShift64s."""
    hidden, inter, group = 2048, 512, 64
    words = inter * hidden // 8
    scale_halves = inter * (hidden // group)
    a, b = [], []
    for _ in range(3):
        w = (rng.next_u64(words) & np.uint64(0xFFFFFFFF)).astype(np.uint32) & np.uint32(0x77777777)
        a.append(w.view(np.uint8))
        p = np.zeros(words, np.uint32)
        for i in range(8):
            p |= ((w >> np.uint32(4 * i)) & np.uint32(7)) << np.uint32(3 * i)
        b.append(p.view(np.uint8).reshape(-1, 4)[:, :3].ravel())
        # packed_3bit.rs:36-38 converts to bf16 by truncation (bits >> 16).
        trunc = lambda v: (np.asarray(v, np.float32).view(np.uint32) >> np.uint32(16)).astype(np.uint16)
        s = trunc(np.float32(0.01) + np.float32(0.02) * np.abs(rng.unit(scale_halves)))
        bi = trunc(np.float32(0.02) * rng.unit(scale_halves))
        sb = np.concatenate([s.view(np.uint8), bi.view(np.uint8)])
        a.append(sb)
        b.append(sb)
    return np.concatenate(a), np.concatenate(b)
