"""Pins the CPU oracle (oracle/oracle.c) to the reference.

Each oracle function is checked against something other than itself:
the reference's own known-answer tests (file:line cited), closed forms,
hand-derived sequential-float results, float64 brute force, and
invariants between independent restatements. CPU only.
"""
import math

import numpy as np
import pytest

import oracle
from helpers import dequant_f64, expert_f64, gen_expert_blob, gen_quant_matrix, q4_block_views, rel_err


# --- cpu_matvec.rs KATs -------------------------------------------------------

def test_dequant_matvec_all_ones():
    """cpu_matvec.rs:486-498: nibbles 1, scale 1, bias 0, x = 1 -> 64.0."""
    rc, out = oracle.dequant_matvec_4bit_gs(np.full(8, 0x11111111, np.uint32), np.array([0x3F80], np.uint16),
                                           np.array([0], np.uint16), 64, 1, 64, np.ones(64, np.float32))
    assert rc == 0 and out[0] == 64.0


def test_zero_input_yields_zero_output():
    """cpu_matvec.rs:519-534."""
    rc, out = oracle.dequant_matvec_4bit_gs(np.full(16, 0xFFFFFFFF, np.uint32), np.full(2, 0x3F80, np.uint16),
                                           np.full(2, 0x3F80, np.uint16), 64, 2, 64, np.zeros(64, np.float32))
    assert rc == 0 and list(out) == [0.0, 0.0]


def test_bias_only_path():
    """cpu_matvec.rs:539-554: nibble 0, scale 5, bias 2 -> 128.0."""
    rc, out = oracle.dequant_matvec_4bit_gs(np.zeros(8, np.uint32), np.array([0x40A0], np.uint16),
                                           np.array([0x4000], np.uint16), 64, 1, 64, np.ones(64, np.float32))
    assert rc == 0 and out[0] == 128.0


def test_in_dim_alignment_check():
    """cpu_matvec.rs:663-674: in_dim 65 -> InDimNotMultiple."""
    rc, _ = oracle.dequant_matvec_4bit_gs(np.zeros(9, np.uint32), np.array([0x3F80], np.uint16),
                                         np.array([0], np.uint16), 65, 1, 64, np.ones(65, np.float32))
    assert rc == 1


def test_matvec_sequential_fma_order():
    """Pins the per-row order: acc = fma(w, x, acc) over c in order
    (cpu_matvec.rs:160-168). With w = 1 and x = [2^24, 1, -2^24, 1, ...]
    the in-order sum is exactly 31 (the first 1 is absorbed by 2^24, each
    later 1 after the cancellation survives); a pairwise or reversed sum
    gives a different value."""
    x = np.zeros(64, np.float32)
    x[0], x[1], x[2] = 2.0**24, 1.0, -(2.0**24)
    x[3:] = 0.0
    x[3:34] = 1.0
    rc, out = oracle.dequant_matvec_4bit_gs(np.full(8, 0x11111111, np.uint32), np.array([0x3F80], np.uint16),
                                           np.array([0], np.uint16), 64, 1, 64, x)
    assert rc == 0 and out[0] == 31.0


def test_dequant_closed_form_all_codes():
    """w = fma(q, s, b) with one rounding (cpu_matvec.rs:164-165). In float64
    q*s and q*s + b are exact for these bf16 operands, so the single f32
    rounding of the float64 value is the fused result."""
    rng = np.random.default_rng(1)
    s = oracle.f32_to_bf16(np.abs(rng.standard_normal(64)) * 0.02)
    b = oracle.f32_to_bf16(rng.standard_normal(64) * 0.01)
    # Row r: all 16 codes twice, group r.
    word = np.uint32(sum(i << (4 * i) for i in range(8)))
    word2 = np.uint32(sum((8 + i) << (4 * i) for i in range(8)))
    packed = np.tile(np.array([word, word2] * 4, np.uint32), 64)
    w = oracle.dequant_4bit(packed, s, b, 64, 64, 64)
    q = np.tile(np.arange(16, dtype=np.float64), 4)
    want = (q[None, :] * oracle.bf16_to_f32(s).astype(np.float64)[:, None]
            + oracle.bf16_to_f32(b).astype(np.float64)[:, None]).astype(np.float32)
    assert np.array_equal(w.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("out_dim,in_dim,group", [(64, 256, 64), (48, 512, 32), (16, 2048, 128)])
def test_matvec_vs_f64_bruteforce(out_dim, in_dim, group):
    rng = np.random.default_rng(out_dim + in_dim)
    codes, s, b = gen_quant_matrix(rng, out_dim, in_dim, group)
    x = rng.standard_normal(in_dim).astype(np.float32)
    rc, out = oracle.dequant_matvec_4bit_gs(codes.view(np.uint32), s, b, in_dim, out_dim, group, x)
    assert rc == 0
    want = dequant_f64(codes.view(np.uint32), s, b, in_dim, out_dim, group) @ x.astype(np.float64)
    assert rel_err(out, want) < 1e-5


def test_matvec_thread_count_invariant():
    rng = np.random.default_rng(7)
    codes, s, b = gen_quant_matrix(rng, 333, 512, 64)
    x = rng.standard_normal(512).astype(np.float32)
    outs = [oracle.dequant_matvec_4bit_gs(codes.view(np.uint32), s, b, 512, 333, 64, x, n)[1] for n in (1, 3, 8)]
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


def test_lm_head_same_arithmetic_as_matvec():
    """lm_head.rs:66-122 is cpu_matvec's arithmetic, single-threaded."""
    rng = np.random.default_rng(3)
    codes, s, b = gen_quant_matrix(rng, 200, 2048, 64)
    x = rng.standard_normal(2048).astype(np.float32)
    a = oracle.lm_head(codes.view(np.uint32), s, b, 2048, 200, 64, x)
    _, m = oracle.dequant_matvec_4bit_gs(codes.view(np.uint32), s, b, 2048, 200, 64, x)
    assert np.array_equal(a, m)


def test_f32_matvec_vs_f64():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((64, 2048)) * 0.02).astype(np.float32)
    x = rng.standard_normal(2048).astype(np.float32)
    assert rel_err(oracle.f32_matvec(w, x), w.astype(np.float64) @ x.astype(np.float64)) < 1e-5


# --- layout (variants.rs) ---------------------------------------------------------

def test_expert_bytes_reference_sizes():
    """Blob sizes at the BASELINE shapes (variants.rs:519-528)."""
    assert oracle.expert_bytes(2048, 1024, 4, 64) == 3_538_944   # OLMoE
    assert oracle.expert_bytes(2048, 512, 4, 64) == 1_769_472    # Qwen3.6-A3B
    assert oracle.expert_bytes(2048, 512, 3, 64) == 1_376_256    # packed 3-bit
    assert oracle.expert_offsets(2048, 512, 4, 64, 1) == (589_824, 589_824 + 524_288, 589_824 + 524_288 + 32_768)


# --- 3-bit layout ---------------------------------------------------------------

def test_pack_3bit_matches_reference_test_packer_and_roundtrips():
    """pack_weights (tools/pack_experts.py:41-54) agrees with the packer
    written independently in packed_3bit.rs:44-51 (p |= (w>>4i & 7) << 3i,
    low 3 bytes), and q3_expert_to_q4 (moe_cpu.rs:227-245) inverts it."""
    rng = np.random.default_rng(5)
    hidden, inter, group = 256, 64, 64
    blob4 = gen_expert_blob(rng, hidden, inter, group, 4)
    # Make every code 3-bit.
    for blk in range(3):
        w, s, _ = oracle.expert_offsets(hidden, inter, 4, group, blk)
        blob4[w:s] &= 0x77
    blob3 = []
    for blk in range(3):
        w, s, _ = oracle.expert_offsets(hidden, inter, 4, group, blk)
        words = blob4[w:s].view(np.uint32)
        packed = oracle.pack_3bit(words)
        p = np.zeros(words.size, np.uint32)
        for i in range(8):
            p |= ((words >> np.uint32(4 * i)) & np.uint32(7)) << np.uint32(3 * i)
        assert np.array_equal(packed, p.view(np.uint8).reshape(-1, 4)[:, :3].ravel())
        sb_end = oracle.expert_offsets(hidden, inter, 4, group, blk + 1)[0] if blk < 2 else blob4.size
        blob3 += [packed, blob4[s:sb_end]]
    blob3 = np.concatenate(blob3)
    assert blob3.size == oracle.expert_bytes(hidden, inter, 3, group)
    assert np.array_equal(oracle.q3_expert_to_q4(blob3, hidden, inter, group), blob4)


# --- expert FFN (moe_cpu.rs:178-220) -------------------------------------------------

@pytest.mark.parametrize("hidden,inter,group", [(256, 128, 64), (512, 64, 32)])
def test_expert_swiglu_vs_f64(hidden, inter, group):
    rng = np.random.default_rng(hidden + inter)
    blob = gen_expert_blob(rng, hidden, inter, group, 4)
    x = rng.standard_normal(hidden).astype(np.float32)
    out = oracle.expert_swiglu(blob, 4, hidden, inter, group, x)
    assert rel_err(out, expert_f64(blob, hidden, inter, group, x)) < 1e-4


def test_expert_swiglu_3bit_equals_repacked_4bit():
    """A 3-bit blob computes exactly what its 4-bit rewrite does
    (backend/cpu/mod.rs:1147-1157)."""
    rng = np.random.default_rng(9)
    hidden, inter, group = 256, 64, 64
    blob3 = gen_expert_blob(rng, hidden, inter, group, 3)
    x = rng.standard_normal(hidden).astype(np.float32)
    a = oracle.expert_swiglu(blob3, 3, hidden, inter, group, x)
    b = oracle.expert_swiglu(oracle.q3_expert_to_q4(blob3, hidden, inter, group), 4, hidden, inter, group, x)
    assert np.array_equal(a, b)


# --- router (moe_router.rs KATs) ---------------------------------------------------------

def test_softmax_normalizes_to_one():
    """moe_router.rs:443-449."""
    assert abs(float(np.sum(oracle.softmax([1.0, 2.0, 3.0, 4.0]))) - 1.0) < 1e-6


def test_softmax_vs_f64():
    rng = np.random.default_rng(11)
    v = rng.standard_normal(256).astype(np.float32)
    e = np.exp(v.astype(np.float64) - v.max())
    assert rel_err(oracle.softmax(v), e / e.sum()) < 1e-6


def test_topk_picks_largest():
    """moe_router.rs:451-462, plus the hand-derived slot order [3, 1, 2]:
    0.9 (index 3) replaces the running minimum 0.1 in slot 0."""
    rc, idx, val = oracle.topk([0.1, 0.5, 0.3, 0.9, 0.2], 3)
    assert rc == 0 and list(idx) == [3, 1, 2]
    assert list(val) == [np.float32(0.9), np.float32(0.5), np.float32(0.3)]


@pytest.mark.parametrize("scores,k,want", [
    ([1.0, 1.0, 1.0, 1.0], 2, [0, 1]),     # equal scores never replace (strict >)
    ([2.0, 1.0, 1.0, 3.0], 2, [0, 3]),     # 3 replaces the minimum slot 1
    ([1.0, 1.0, 2.0], 2, [2, 1]),          # tie between slots: the lower slot is replaced
    ([5.0, 4.0, 3.0, 2.0, 1.0], 5, [0, 1, 2, 3, 4]),
])
def test_topk_hand_derived_ties(scores, k, want):
    assert list(oracle.topk(scores, k)[1]) == want


def test_topk_bad_k():
    assert oracle.topk([1.0, 2.0], 0)[0] == 2
    assert oracle.topk([1.0, 2.0], 3)[0] == 2


def test_topk_set_vs_sort():
    """Distinct scores: the chosen set is the k largest."""
    rng = np.random.default_rng(12)
    for _ in range(20):
        v = rng.standard_normal(256).astype(np.float32)
        _, idx, val = oracle.topk(v, 8)
        assert set(idx) == set(np.argsort(-v)[:8])
        assert np.array_equal(val, v[idx])


def test_router_without_renorm_keeps_softmax_probs():
    """moe_router.rs:467-493 (norm_topk_prob false keeps raw probs, picks
    {2, 4}; true renormalises the same picks by * (1 / sum))."""
    logits = [0.5, -1.0, 2.0, 0.0, 1.5, -0.5]
    probs = oracle.softmax(logits)
    rc, raw_idx, raw_w = oracle.router(logits, 2, False)
    assert rc == 0 and sorted(raw_idx) == [2, 4]
    for s in range(2):
        assert raw_w[s] == probs[raw_idx[s]]
    assert raw_w.sum() < 1.0
    _, norm_idx, norm_w = oracle.router(logits, 2, True)
    assert list(norm_idx) == list(raw_idx)
    total = np.float32(raw_w[0] + raw_w[1])
    for s in range(2):
        assert norm_w[s] == np.float32(raw_w[s] * np.float32(np.float32(1.0) / total))


def test_normalize_sums_to_one():
    """moe_router.rs:495-501."""
    assert abs(float(oracle.normalize_weights([0.5, 1.5, 2.0]).sum()) - 1.0) < 1e-6


def test_normalize_guard():
    assert list(oracle.normalize_weights([0.0, 0.0])) == [0.0, 0.0]


# --- noaux_tc router (moe_router.rs:211-330) -----------------------------------------------

def test_noaux_tc_hand_reference():
    """moe_router.rs:528-580: group 1 wins (top-2 sums 2.3128 vs 2.1317 of
    biased sigmoid scores), idx set {5, 7}, weights gather the UN-biased
    sigmoid 0.8808 / 0.9820, renormalised and * 2.5 -> 1.1822 / 1.3178."""
    logits = [3.0, -2.0, 1.0, -1.0, -3.0, 2.0, 0.0, 4.0]
    bias = [0.1, 0.2, -0.3, 0.0, 0.0, 0.4, -0.1, 0.05]
    rc, idx, w, s = oracle.noaux_tc_router(logits, bias, 2, 1, 2, 2.5)
    assert rc == 0
    pairs = sorted(zip(idx.tolist(), w.tolist()))
    assert [i for i, _ in pairs] == [5, 7]
    assert abs(pairs[0][1] - 1.1822) < 1e-3 and abs(pairs[1][1] - 1.3178) < 1e-3
    assert abs(float(w.sum()) - 2.5) < 1e-3
    # The logits are left holding the un-biased sigmoid scores.
    assert all(s[i] == np.float32(oracle.sigmoid(x)) for i, x in enumerate(logits))


def test_noaux_tc_cogito_shape():
    """moe_router.rs:585-640 (256 experts, 8 groups, top-4 groups, k 8,
    scaling 2.5, logits sin(0.137 i) * 2, bias cos(0.241 i) * 0.5)."""
    i = np.arange(256, dtype=np.float32)
    logits = (np.sin(i * np.float32(0.137)) * 2).astype(np.float32)
    bias = (np.cos(i * np.float32(0.241)) * np.float32(0.5)).astype(np.float32)
    rc, idx, w, _ = oracle.noaux_tc_router(logits, bias, 8, 4, 8, 2.5)
    assert rc == 0
    assert abs(float(w.sum()) - 2.5) < 1e-3
    assert len({int(j) // 32 for j in idx}) <= 4
    assert len(set(idx.tolist())) == 8


def _noaux_f64(logits, bias, n_group, topk_group, k, scale):
    """Independent restatement by sorting, in float64 (distinct values)."""
    s = 1.0 / (1.0 + np.exp(-np.asarray(logits, np.float64)))
    b = s + np.asarray(bias, np.float64)
    g = b.reshape(n_group, -1)
    gsc = np.sort(g, axis=1)[:, -2:].sum(axis=1) if g.shape[1] > 1 else g[:, 0] + -np.inf
    keep = np.argsort(-gsc, kind="stable")[:topk_group]
    m = np.full_like(b, -np.inf)
    gs = b.size // n_group
    for gi in keep:
        m[gi * gs:(gi + 1) * gs] = b[gi * gs:(gi + 1) * gs]
    sel = np.argsort(-m, kind="stable")[:k]
    return set(sel.tolist()), {int(j): s[j] / s[sel].sum() * scale for j in sel}


@pytest.mark.parametrize("n,n_group,topk_group,k", [(256, 8, 4, 8), (64, 4, 2, 6), (512, 16, 3, 10),
                                                    (128, 1, 1, 8), (96, 3, 3, 4)])
def test_noaux_tc_vs_sort_f64(n, n_group, topk_group, k):
    rng = np.random.default_rng(n + k)
    for _ in range(10):
        logits = rng.standard_normal(n).astype(np.float32) * 2
        bias = rng.standard_normal(n).astype(np.float32) * 0.3
        rc, idx, w, _ = oracle.noaux_tc_router(logits, bias, n_group, topk_group, k, 2.5)
        want_set, want_w = _noaux_f64(logits, bias, n_group, topk_group, k, 2.5)
        assert rc == 0 and set(idx.tolist()) == want_set
        for j, wj in zip(idx.tolist(), w.tolist()):
            assert abs(wj - want_w[j]) <= 1e-6 * 2.5


def test_noaux_tc_group_score_is_top2_sum():
    """Group 0 holds the single largest score (sigmoid 3 = 0.9526) but its
    top-2 sum 1.0 loses to group 1's 0.7311 * 2: the winner is expert 2 (the
    earlier of the tied pair: a later equal value never replaces)."""
    rc, idx, w, _ = oracle.noaux_tc_router([3.0, -3.0, 1.0, 1.0], [0.0] * 4, 2, 1, 1, 1.5)
    assert rc == 0 and list(idx) == [2] and w[0] == np.float32(1.5)


def test_noaux_tc_bias_selects_but_does_not_weight():
    """Un-biased, the top-2 would be {0, 2}; the bias lifts expert 1
    (0.2689 + 0.6) above expert 0 (0.5), and expert 2 (0.6225) then replaces
    slot 0: idx [2, 1]. The weights still gather the un-biased scores."""
    rc, idx, w, _ = oracle.noaux_tc_router([0.0, -1.0, 0.5], [0.0, 0.6, 0.0], 1, 1, 2, 1.0)
    assert rc == 0 and list(idx) == [2, 1]
    s1, s2 = 1.0 / (1.0 + math.exp(1.0)), 1.0 / (1.0 + math.exp(-0.5))
    assert abs(w[0] - s2 / (s1 + s2)) < 1e-6 and abs(w[1] - s1 / (s1 + s2)) < 1e-6


def test_noaux_tc_more_slots_than_unmasked_experts():
    """k = 3 with one kept group of 2 experts: the third slot keeps the
    reference's start entry (index 0), so its weight gathers sigmoid(3)."""
    rc, idx, w, _ = oracle.noaux_tc_router([3.0, -3.0, 1.0, 1.0], [0.0] * 4, 2, 1, 3, 1.0)
    assert rc == 0 and list(idx) == [2, 3, 0]
    s = [1.0 / (1.0 + math.exp(-x)) for x in (1.0, 1.0, 3.0)]
    for got, want in zip(w, s):
        assert abs(got - want / sum(s)) < 1e-6


@pytest.mark.parametrize("n,n_group,topk_group,k,rc", [
    (0, 1, 1, 1, 3), (8, 0, 1, 1, 2), (8, 3, 1, 1, 2), (8, 2, 0, 1, 2), (8, 2, 3, 1, 2),
    (8, 2, 1, 0, 2), (8, 2, 1, 9, 2),
])
def test_noaux_tc_errors(n, n_group, topk_group, k, rc):
    """moe_router.rs:221-255: EmptyScores, then BadK for the group count, the
    kept-group count and k."""
    assert oracle.noaux_tc_router([0.0] * n, [0.0] * n, n_group, topk_group, k, 1.0)[0] == rc


# --- combine (deferred.rs:441-490) ---------------------------------------------------------

def test_combine_known_answers():
    out = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    w = np.array([0.5, 0.25], np.float32)
    h_mid = np.array([10.0, 20.0], np.float32)
    # moe = [0.5 + 0.75, 1 + 1] = [1.25, 2.0]
    assert list(oracle.combine(out, w, h_mid)) == [11.25, 22.0]
    # sigmoid(0) = 0.5 exactly: + 0.5 * shared
    sh = np.array([2.0, 4.0], np.float32)
    assert list(oracle.combine(out, w, h_mid, sh, 0.0)) == [12.25, 24.0]
    # NaN score: unscaled shared add
    assert list(oracle.combine(out, w, h_mid, sh)) == [13.25, 26.0]
    assert oracle.sigmoid(0.0) == 0.5


def test_rms_norm_vs_f64():
    rng = np.random.default_rng(13)
    x = rng.standard_normal(2048).astype(np.float32)
    w = oracle.f32_to_bf16(1.0 + 0.1 * rng.standard_normal(2048))
    got = oracle.rms_norm_bf16(x, w, 1e-6)
    xd = x.astype(np.float64)
    want = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * oracle.bf16_to_f32(w)
    assert rel_err(got, want) < 1e-6


# --- decode layer composition ---------------------------------------------------------

def test_decode_layer_is_router_experts_combine():
    """orc_moe_decode_layer wires the pieces: f32 router logits ->
    moe_router_cpu_with -> expert FFN per slot -> shared + sigmoid gate ->
    cpu_combine. Compared with the pieces called one by one (exact) and
    with a float64 brute force of the whole layer."""
    rng = np.random.default_rng(21)
    H, I, E, k, G = 256, 64, 16, 4, 64
    blobs = [gen_expert_blob(rng, H, I, G, 4) for _ in range(E)]
    stride = blobs[0].size
    experts = np.concatenate(blobs)
    shared = gen_expert_blob(rng, H, I, G, 4)
    router_w = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    gate_w = (rng.standard_normal(H) * 0.02).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    h_mid = rng.standard_normal(H).astype(np.float32)
    out, idx, w, logits = oracle.moe_decode_layer(experts, stride, H, I, E, k, G, 4, True, router_w, x, h_mid,
                                                  shared, gate_w)
    lg = oracle.f32_matvec(router_w, x)
    assert np.array_equal(lg, logits)
    _, idx2, w2 = oracle.router(lg, k, True)
    assert np.array_equal(idx, idx2) and np.array_equal(w, w2)
    outs = np.stack([oracle.expert_swiglu(blobs[e], 4, H, I, G, x) for e in idx])
    sh = oracle.expert_swiglu(shared, 4, H, I, G, x)
    score = oracle.f32_matvec(gate_w[None, :], x)[0]
    assert np.array_equal(out, oracle.combine(outs, w, h_mid, sh, score))
    # float64 brute force of the layer with the same picks.
    want = h_mid.astype(np.float64)
    for s, e in enumerate(idx):
        want = want + float(w[s]) * expert_f64(blobs[e], H, I, G, x)
    g = float(gate_w.astype(np.float64) @ x.astype(np.float64))
    want = want + expert_f64(shared, H, I, G, x) / (1.0 + math.exp(-g))
    assert rel_err(out, want) < 1e-4


# --- prefill buckets (moe_router.rs KATs) ------------------------------------------------

def test_build_expert_buckets_round_trips():
    """moe_router.rs:645-685."""
    idx = [0, 3, 0, 2, 3, 0]
    w = [0.7, 0.3, 0.4, 0.6, 0.5, 0.5]
    rc, eids, offs, tok, ws = oracle.build_expert_buckets(idx, w, 3, 2, 4)
    assert rc == 0 and list(eids) == [0, 2, 3] and list(offs) == [0, 3, 4, 6]
    got = {t: [] for t in range(3)}
    for b, e in enumerate(eids):
        for j in range(offs[b], offs[b + 1]):
            got[int(tok[j])].append((int(e), float(ws[j])))
    for t in range(3):
        want = sorted((idx[t * 2 + s], np.float32(w[t * 2 + s])) for s in range(2))
        assert sorted(got[t]) == [(e, float(v)) for e, v in want]


def test_build_expert_buckets_distinct_tokens_per_bucket():
    """moe_router.rs:690-706."""
    _, eids, offs, tok, _ = oracle.build_expert_buckets([0, 1, 1, 2, 0, 2, 1, 3], [0.5] * 8, 4, 2, 4)
    for b in range(len(eids)):
        t = list(tok[offs[b]:offs[b + 1]])
        assert len(set(t)) == len(t)


def test_build_expert_buckets_empty_skipped():
    """moe_router.rs:710-725."""
    _, eids, offs, tok, _ = oracle.build_expert_buckets([2, 7, 7, 2], [0.5] * 4, 2, 2, 10)
    assert list(eids) == [2, 7] and list(offs) == [0, 2, 4]
    assert sorted(tok[0:2]) == [0, 1] and sorted(tok[2:4]) == [0, 1]


def test_build_expert_buckets_single_expert():
    """moe_router.rs:729-737."""
    _, eids, offs, tok, ws = oracle.build_expert_buckets([3, 3, 3, 3], [1.0] * 4, 4, 1, 8)
    assert list(eids) == [3] and list(offs) == [0, 4] and list(tok) == [0, 1, 2, 3]
    assert list(ws) == [1.0] * 4


def test_permute_fuse_matches_tokenwise():
    """batched_diff_oracle.rs:893-1000: 4 tokens x 4 slots over 12 experts
    (4 empty), bucket order vs token order; and float64 brute force."""
    rng = np.random.default_rng(0xCAFE)
    H, I, G = 256, 64, 64
    routing = np.array([[0, 1, 2, 3], [2, 3, 4, 5], [4, 5, 6, 7], [6, 7, 0, 1]], np.int32)
    weights = (rng.random((4, 4)) * 0.4 + 0.3).astype(np.float32)
    x = rng.uniform(-1, 1, (4, H)).astype(np.float32)
    blobs = [gen_expert_blob(rng, H, I, G, 4) for _ in range(12)]
    stride = blobs[0].size
    experts = np.concatenate(blobs)
    buckets = oracle.build_expert_buckets(routing, weights, 4, 4, 12)
    assert list(buckets[1]) == list(range(8))
    out = oracle.moe_permute_fuse(experts, stride, 4, H, I, G, x, buckets, 4)
    for t in range(4):
        tokenwise = np.zeros(H, np.float32)
        want = np.zeros(H)
        for s in range(4):
            e = routing[t, s]
            y = oracle.expert_swiglu(blobs[e], 4, H, I, G, x[t])
            tokenwise = tokenwise + weights[t, s] * y
            want += float(weights[t, s]) * expert_f64(blobs[e], H, I, G, x[t])
        cos = float(np.dot(out[t], tokenwise) / (np.linalg.norm(out[t]) * np.linalg.norm(tokenwise)))
        assert cos >= 0.9999
        assert rel_err(out[t], want) < 1e-4


def test_xorshift_stream_known_values():
    """xorshift64* of the reference tests; first outputs of seed 1 computed
    by hand from the recurrence in Python integers."""
    st = 1
    want = []
    for _ in range(3):
        st ^= st >> 12
        st ^= (st << 25) & 0xFFFFFFFFFFFFFFFF
        st ^= st >> 27
        want.append((st * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF)
    assert [int(v) for v in oracle.XorShift64s(1).next_u64(3)] == want


@pytest.mark.parametrize("pos", [0, 3, 255])
def test_router_nan_logit_keeps_start_slots(pos):
    """moe_router.rs:52-141 with one NaN logit: the softmax sum is NaN, so
    every probability is NaN; `score > values[min_k]` is then never true,
    all k slots keep their start (index 0, -1e30), and the guarded
    renormalisation (sum > 0 fails) leaves the weights as they are. The
    position of the NaN does not matter (a NaN at index 0 becomes the max
    and poisons every exp; elsewhere it poisons the sum)."""
    rng = np.random.default_rng(pos)
    logits = rng.standard_normal(256).astype(np.float32)
    logits[pos] = np.nan
    probs = oracle.softmax(logits)
    assert np.all(np.isnan(probs))
    for normalize in (False, True):
        rc, idx, w = oracle.router(logits, 8, normalize)
        assert rc == 0
        assert np.all(idx == 0)
        assert np.all(w == np.float32(-1e30))


def test_argmax_is_the_reference_scan_with_nan():
    """orc_argmax is the reference's greedy fold (engine_tests.rs:105-107):
    first maximal index, NaN never replaces the best, a NaN at index 0 is
    kept (every comparison with it is false)."""
    v = np.array([np.nan, 3.0, 5.0, 5.0, 1.0], np.float32)
    assert oracle.argmax(v) == 0
    v = np.array([1.0, np.nan, 5.0, np.nan, 5.0], np.float32)
    assert oracle.argmax(v) == 2
    v = np.full(7, np.nan, np.float32)
    assert oracle.argmax(v) == 0
    v = np.array([-np.inf, -np.inf], np.float32)
    assert oracle.argmax(v) == 0


# ---- prefill MoE block tail: moe_combine_residual_n_tokens_cpu ------------------
def test_combine_residual_n_tokens_known_answers():
    """backend/cpu/mod.rs:657-695: hidden = h_mid + moe_sum + sigmoid(g) *
    shared; sigmoid(0) = 0.5 exactly (exp(-0) = 1)."""
    h = np.array([[1.0, -2.0]], np.float32)
    m = np.array([[2.0, 0.5]], np.float32)
    s = np.array([[4.0, 8.0]], np.float32)
    out = oracle.moe_combine_residual_n_tokens(h, m, s, np.zeros(1, np.float32))
    assert np.array_equal(out, np.array([[5.0, 2.5]], np.float32))
    # no shared expert: h_mid + moe_sum
    assert np.array_equal(oracle.moe_combine_residual_n_tokens(h, m), np.array([[3.0, -1.5]], np.float32))
    # no gate: the shared term unscaled
    assert np.array_equal(oracle.moe_combine_residual_n_tokens(h, m, s), np.array([[7.0, 6.5]], np.float32))


def test_combine_residual_n_tokens_addition_order():
    """Left to right, (h_mid + moe_sum) + g * shared: with h_mid = 1e8,
    moe_sum = -1e8 and g * shared = 1 the result is 1; summing the other
    way, h_mid + (moe_sum + 1) rounds -1e8 + 1 back to -1e8 and gives 0."""
    h = np.array([[1e8]], np.float32)
    m = np.array([[-1e8]], np.float32)
    s = np.array([[2.0]], np.float32)
    out = oracle.moe_combine_residual_n_tokens(h, m, s, np.zeros(1, np.float32))
    assert out[0, 0] == np.float32(1.0)
    assert np.float32(h[0, 0] + np.float32(m[0, 0] + np.float32(1.0))) == np.float32(0.0)


def test_combine_residual_n_tokens_no_fused_multiply_add():
    """g * shared is rounded before the add (Rust does not contract): on
    inputs where fma(g, s, a) and a + round(g * s) differ, the oracle gives
    the latter."""
    rng = np.random.default_rng(11)
    found = 0
    for _ in range(2000):
        gate = np.float32(rng.uniform(-3, 3))
        g = np.float32(oracle.sigmoid(float(gate)))
        s = np.float32(rng.uniform(0.5, 2.0))
        a = -np.float32(np.float64(g) * np.float64(s))  # cancels the product to about one ulp
        fused = np.float32(np.float64(a) + np.float64(g) * np.float64(s))
        unfused = np.float32(a + np.float32(g * s))
        if fused == unfused:
            continue
        found += 1
        out = oracle.moe_combine_residual_n_tokens(np.array([[a]], np.float32), np.zeros((1, 1), np.float32),
                                                   np.array([[s]], np.float32), np.array([gate], np.float32))
        assert out[0, 0] == unfused and out[0, 0] != fused
    assert found >= 20


def test_combine_residual_n_tokens_vs_f64():
    rng = np.random.default_rng(12)
    n, d = 7, 300
    h, m, s = (rng.standard_normal((n, d)).astype(np.float32) for _ in range(3))
    gate = rng.standard_normal(n).astype(np.float32)
    out = oracle.moe_combine_residual_n_tokens(h, m, s, gate)
    g64 = 1.0 / (1.0 + np.exp(-gate.astype(np.float64)))
    want = h.astype(np.float64) + m + g64[:, None] * s
    assert rel_err(out, want) <= 1e-6
