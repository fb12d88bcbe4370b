"""The oracle's MoE-router restatement (deltanet.metal:863-900, 2229-2329)
pinned without the reference: the Q8 closed form bit for bit against numpy's
byte view, the factored logits against an fp64 dense product, and the top-8
rule against numpy's stable descending sort (ties keep the lower index) and
a direct fp64 softmax over the eight."""
import numpy as np

from oracle import oracle as O
from qff import synth


def test_q8_dequant_closed_form():
    w, s, b = synth.q8_weight(7, 192, seed=1)
    got = O.q8_dequant(w, s, b, O.BF16)
    q = w.view(np.uint8).reshape(7, 192).astype(np.float32)   # little-endian: byte c = element c
    sc = np.repeat(O.bf16_to_f32(s), 64, axis=1)
    bi = np.repeat(O.bf16_to_f32(b), 64, axis=1)
    assert np.array_equal(got.view(np.uint32), (q * sc + bi).astype(np.float32).view(np.uint32))


def test_q8_dequant_special_words():
    w = np.array([[0x00000000] * 16, [0xFFFFFFFF] * 16, [0x04030201] * 16], np.uint32)
    s = O.f32_to_f16(np.full((3, 1), 0.5, np.float32))
    b = O.f32_to_f16(np.full((3, 1), -1.0, np.float32))
    got = O.q8_dequant(w, s, b, O.F16)
    assert np.all(got[0] == -1.0) and np.all(got[1] == 255 * 0.5 - 1.0)
    assert np.array_equal(got[2][:4], np.array([1, 2, 3, 4], np.float32) * 0.5 - 1.0)


def test_router_logits_match_fp64():
    w, s, b = synth.q8_weight(256, 2048, seed=2)
    x = np.random.default_rng(3).standard_normal(2048).astype(np.float32)
    got = O.router_logits(w, s, b, x, O.BF16)
    ref = O.q8_dequant(w, s, b, O.BF16).astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref)) + 1e-5


def _top8_ref(lg):
    order = np.argsort(-lg.astype(np.float64), kind="stable")[:8]
    top = lg[order].astype(np.float64)
    p = np.exp(top - top[0])
    return order, p / p.sum()


def test_router_top8_matches_sort_and_softmax():
    rng = np.random.default_rng(4)
    for n in (256, 64, 8):
        lg = (rng.standard_normal(n) * 3).astype(np.float32)
        idx, sc = O.router_top8(lg)
        ref_i, ref_s = _top8_ref(lg)
        assert np.array_equal(idx, ref_i)
        assert np.allclose(sc, ref_s, atol=1e-6)
        assert abs(float(sc.sum()) - 1.0) < 1e-6


def test_router_top8_ties_keep_lower_index():
    lg = np.zeros(256, np.float32)
    lg[[200, 3, 77, 150]] = 5.0        # four equal maxima
    lg[[10, 11]] = 4.0
    idx, sc = O.router_top8(lg)
    assert list(idx[:6]) == [3, 77, 150, 200, 10, 11]
    assert list(idx[6:]) == [0, 1]     # then the zeros by index
    assert np.allclose(sc[:4], sc[0]) and np.allclose(sc[6:], sc[6])
