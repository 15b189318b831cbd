"""Host-side pieces of the privacy-filter model (runntime_amd/
privacy_filter.py): the constrained Viterbi decoder (native, and the
oracle's numpy restatement) against brute force over every label path
(viterbi.ts:20-148 defines the best-scoring valid path),
the label info (config.ts:1-75), token spans (spans.ts:18-70), the YaRN
rope tables at their closed-form limits (rope.ts:24-94) and log-softmax."""
import itertools
import math

import numpy as np
import pytest

from oracle import ref
from runntime_amd import privacy_filter as pf


def test_label_info():
    info = pf.build_label_info(pf.V2_NER_CLASS_NAMES)
    assert info.num_classes == 33 and len(info.span_class_names) == 9
    assert info.background_token_label == 0
    assert pf.V2_NER_CLASS_NAMES[1:5] == ["B-account_number", "I-account_number",
                                          "E-account_number", "S-account_number"]
    assert info.token_boundary_tags[4] == "S" and info.token_to_span_label[4] == 1


def _brute(dec, lp):
    T, n = lp.shape
    best, arg = -np.inf, None
    for path in itertools.product(range(n), repeat=T):
        s = dec.start[path[0]] + lp[0, path[0]] + dec.end[path[-1]]
        for t in range(1, T):
            s += dec.trans[path[t - 1], path[t]] + lp[t, path[t]]
        if s > best:
            best, arg = s, list(path)
    return arg


@pytest.mark.parametrize("biases", [None, pf.ViterbiBiases(0.3, -0.2, 0.5, -0.1, 0.2, -0.4)])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_viterbi_is_the_best_valid_path(biases, seed):
    info = pf.build_label_info(pf.V2_NER_CLASS_NAMES)
    dec = pf.ViterbiDecoder(info, biases)
    rng = np.random.default_rng(seed)
    lp = pf.log_softmax_rows(rng.standard_normal((3, 33)).astype(np.float32) * 3)
    want = _brute(dec, lp.astype(np.float64))
    assert dec.decode(lp) == want and ref.viterbi_decode(dec.start, dec.end, dec.trans, lp) == want


def test_viterbi_transitions_follow_bioes():
    info = pf.build_label_info(pf.V2_NER_CLASS_NAMES)
    dec = pf.ViterbiDecoder(info)
    B, I, E, S = 1, 2, 3, 4  # account_number
    assert dec.trans[0, B] == 0 and dec.trans[0, I] == dec.NEG_INF
    assert dec.trans[B, I] == 0 and dec.trans[B, E] == 0 and dec.trans[B, 0] == dec.NEG_INF
    assert dec.trans[B, 6] == dec.NEG_INF  # I of another class
    assert dec.trans[E, 0] == 0 and dec.trans[S, 5] == 0
    assert dec.start[I] == dec.NEG_INF and dec.end[B] == dec.NEG_INF


def test_viterbi_rules_for_untagged_and_tagged_background_labels():
    """Labels the v2 class list does not have, worked by hand from the rules
    of viterbi.ts:39-77: a label with tag E but no span class (its moves are
    those of a closed span, with the end biases), a label with a span class
    but no tag (never entered), and a background token that carries span
    class a with tag I (after B-a it continues the span, with the inside
    bias)."""
    info = pf.LabelInfo(
        span_class_names=["O", "a"],
        token_to_span_label={0: 0, 1: 1, 2: 1, 3: 1, 5: 1, 6: 1},
        token_boundary_tags={1: "B", 2: "I", 3: "E", 4: "E", 6: "I"},
        background_token_label=6, background_span_label=0, num_classes=7)
    b = pf.ViterbiBiases(background_stay=1, background_to_start=2, inside_to_continue=3,
                         inside_to_end=4, end_to_background=5, end_to_start=6)
    t = pf.ViterbiDecoder(info, b).trans
    NEG = pf.ViterbiDecoder.NEG_INF
    # 4: tag E, no span class → may be followed by background or B/S
    assert t[4, 0] == 5 and t[4, 6] == 5 and t[4, 1] == 6 and t[4, 2] == NEG and t[4, 3] == NEG
    # 5: span class, no tag → never a next label; as a previous label it
    # opens like background but with no bias
    assert all(t[p, 5] == NEG for p in range(7))
    assert t[5, 0] == 0 and t[5, 1] == 0 and t[5, 2] == NEG
    # 6: the background token, span class a, tag I
    assert t[1, 6] == 3 and t[2, 6] == 3       # continues the open span of class a
    assert t[6, 6] == 1 and t[6, 0] == 1       # background to background
    assert t[6, 1] == 2 and t[6, 2] == NEG     # background to a start only
    assert t[3, 6] == 5 and t[3, 1] == 6       # after E-a


def test_labels_to_spans():
    info = pf.build_label_info(pf.V2_NER_CLASS_NAMES)
    # O B I E O S, then a dangling I and an E without its B
    labels = [0, 1, 2, 3, 0, 8, 10, 0, 7]
    got = [(s.label, s.token_start, s.token_end) for s in pf.labels_to_spans(labels, info)]
    assert got == [(1, 1, 4), (2, 5, 6), (3, 6, 7), (2, 8, 9)]


def test_rope_tables_limits():
    cos, sin = pf.compute_rope_tables(5, 64, 150000.0, 32.0, 1.0, 32.0, 4096)
    conc = 0.1 * math.log(32) + 1
    np.testing.assert_allclose(cos[0], conc, rtol=1e-6)
    np.testing.assert_array_equal(sin[0], 0)
    # dims below the ramp keep 1/freq, dims above it 1/(32·freq)
    freq = 150000.0 ** (2 * np.arange(32) / 64)
    np.testing.assert_allclose(cos[3, 0], math.cos(3 / freq[0]) * conc, rtol=1e-6)
    np.testing.assert_allclose(cos[3, 31], math.cos(3 / (32 * freq[31])) * conc, rtol=1e-6)
    ce, se = pf.rope_constants(5)
    assert ce.shape == (5, 64)
    np.testing.assert_array_equal(ce[:, 0], ce[:, 1])
    np.testing.assert_allclose(ce[0, 0], conc * pf.QK_SCALE, rtol=1e-6)


def test_log_softmax_rows():
    x = np.random.default_rng(0).standard_normal((4, 33)).astype(np.float32)
    lp = pf.log_softmax_rows(x)
    np.testing.assert_allclose(np.exp(lp.astype(np.float64)).sum(1), 1, rtol=1e-6)


@pytest.mark.parametrize("T", [0, 1, 2, 57, 300])
def test_native_viterbi_equals_the_numpy_one(T):
    info = pf.build_label_info(pf.V2_NER_CLASS_NAMES)
    dec = pf.ViterbiDecoder(info, pf.ViterbiBiases(0.1, -0.3, 0.2, 0.0, -0.1, 0.4))
    lp = pf.log_softmax_rows(np.random.default_rng(T).standard_normal((T, 33)).astype(np.float32) * 4
                             ) if T else np.zeros((0, 33), np.float32)
    assert dec.decode(lp) == ref.viterbi_decode(dec.start, dec.end, dec.trans, lp)


def test_native_viterbi_falls_back_to_argmax():
    # every transition forbidden: no finite path, per-token argmax
    info = pf.build_label_info(pf.V2_NER_CLASS_NAMES)
    dec = pf.ViterbiDecoder(info)
    dec.trans[:] = -np.inf
    lp = pf.log_softmax_rows(np.random.default_rng(9).standard_normal((6, 33)).astype(np.float32))
    assert dec.decode(lp) == ref.viterbi_decode(dec.start, dec.end, dec.trans, lp) == [int(j) for j in np.argmax(lp, 1)]


def test_linear_and_attention_argument_checks():
    """Shapes the kernels cannot check from raw pointers are refused on the
    host, before any device call: a Linear's weight and bias, the rope
    tables' rows (moe_attention reads T of them), the sinks."""
    import torch
    from runntime_amd.linear import Linear
    w = torch.zeros((8, 4))
    Linear(8, 4, w, torch.zeros(4))
    with pytest.raises(ValueError, match="bias"):
        Linear(8, 4, w, torch.zeros(5))
    with pytest.raises(ValueError, match="bias"):
        Linear(8, 4, w, torch.zeros(4, dtype=torch.float64))
    with pytest.raises(ValueError, match="weight"):
        Linear(8, 4, torch.zeros((4, 8)).t(), None)
    lin_qkv = Linear(640, 1152, torch.zeros((640, 1152)))
    lin_out = Linear(896, 640, torch.zeros((896, 640)))
    blk = pf.AttnBlock(torch.ones(640), lin_qkv, lin_out, torch.zeros(14))
    x = torch.zeros((10, 640))
    cos, sin = (torch.from_numpy(a) for a in pf.rope_constants(10))
    short = cos[:9].contiguous()
    with pytest.raises(ValueError, match="cos"):
        blk.forward(x, short, sin)
    with pytest.raises(ValueError, match="sin"):
        blk.forward(x, cos, sin.double())
    bad = pf.AttnBlock(torch.ones(640), lin_qkv, lin_out, torch.zeros(13))
    with pytest.raises(ValueError, match="sinks"):
        bad.forward(x, cos, sin)
