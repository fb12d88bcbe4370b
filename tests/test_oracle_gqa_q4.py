"""Pins the full-attention and affine-Q4 halves of the oracle
(deltanet.metal:599-708, 809-861; attention.metal:134-377;
Attention.swift:129-157; QwenQ4ActiveExpertStreamingRunner.swift:899-922,
1090-1099) with closed forms, invariants and brute force."""
import numpy as np
import pytest

from oracle import oracle as O
from qff import synth


def test_head_rmsnorm_closed_form(rng):
    x = rng.standard_normal((16, 256))
    w = rng.standard_normal(256)
    out = O.head_rmsnorm(x, w, prec=64)
    ref = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + 1e-6) * w[None, :]
    assert np.allclose(out, ref, rtol=1e-13)


def test_rope_tables_closed_form():
    for pos in (0, 1, 7, 8191, 65535):
        c, s = O.rope_tables(pos, prec=64)
        i = np.arange(32)
        ang = pos / (1e7 ** (2 * i / 64.0))
        assert np.allclose(c[:32], np.cos(ang), atol=1e-12) and np.array_equal(c[:32], c[32:])
        assert np.allclose(s[:32], np.sin(ang), atol=1e-12) and np.array_equal(s[:32], s[32:])
        c32, s32 = O.rope_tables(pos, prec=32)
        # fp32 host tables (angle = Float(pos) * freq in fp32) stay close
        assert np.max(np.abs(c32 - c)) < 2e-3 and np.max(np.abs(s32 - s)) < 2e-3


def test_rope_identity_at_zero_and_norm_preserving(rng):
    x = rng.standard_normal((4, 256))
    c, s = O.rope_tables(0, prec=64)
    assert np.array_equal(O.rope_partial(x, c, s, prec=64), x)
    c, s = O.rope_tables(1234, prec=64)
    y = O.rope_partial(x, c, s, prec=64)
    assert np.array_equal(y[:, 64:], x[:, 64:])           # only 64 dims rotate
    pair = lambda z: z[:, :32] ** 2 + z[:, 32:64] ** 2     # (i, i+32) pairs
    assert np.allclose(pair(y), pair(x), rtol=1e-12)


def test_rope_relative_position(rng):
    # rotate-half RoPE: <R_p q, R_p' k> depends only on p - p'
    q = rng.standard_normal((1, 256))
    k = rng.standard_normal((1, 256))

    def dot(p, pp):
        cq, sq = O.rope_tables(p, prec=64)
        ck, sk = O.rope_tables(pp, prec=64)
        return float(np.sum(O.rope_partial(q, cq, sq, prec=64) * O.rope_partial(k, ck, sk, prec=64)))

    assert abs(dot(10, 3) - dot(1007, 1000)) < 1e-9
    assert abs(dot(10, 3) - dot(10, 4)) > 1e-6


def np_attention(q, K, V, scale):
    nq, hd = q.shape
    nkv = K.shape[1]
    out = np.zeros((nq, hd))
    for h in range(nq):
        kv = h // (nq // nkv)
        s = K[:, kv, :] @ q[h] * scale
        p = np.exp(s - s.max())
        out[h] = p @ V[:, kv, :] / p.sum()
    return out


@pytest.mark.parametrize("L", [1, 2, 17, 100, 1000])
def test_attention_split_matches_softmax(L, rng):
    q = rng.standard_normal((16, 256))
    K = rng.standard_normal((L, 2, 256))
    V = rng.standard_normal((L, 2, 256))
    ref = np_attention(q, K, V, 1 / 16)
    for nc in (0, 1, 7):                      # reference geometry, single pass, odd split
        out = O.attention_decode(q, K, V, num_chunks=nc, prec=64)
        assert np.allclose(out, ref, rtol=1e-11, atol=1e-12)
    out32 = O.attention_decode(q, K, V, prec=32)
    assert np.max(np.abs(out32 - ref)) < 1e-5


def test_attention_special_cases(rng):
    K = rng.standard_normal((50, 2, 256))
    V = rng.standard_normal((50, 2, 256))
    out = O.attention_decode(np.zeros((16, 256)), K, V, prec=64)      # q = 0 -> mean of V
    assert np.allclose(out[:8], V[:, 0].mean(0)) and np.allclose(out[8:], V[:, 1].mean(0))
    out = O.attention_decode(rng.standard_normal((16, 256)), K[:1], V[:1], prec=64)  # L = 1 -> v
    assert np.allclose(out[:8], V[0, 0]) and np.allclose(out[8:], V[0, 1])


def test_gqa_token_matches_matrix_form(rng):
    p = {k: v.astype(np.float64) for k, v in synth.gqa_params().items()}
    max_seq, pos = 40, 29
    kc = O.f32_to_bf16(rng.standard_normal((max_seq, 2, 256)).astype(np.float32))
    vc = O.f32_to_bf16(rng.standard_normal((max_seq, 2, 256)).astype(np.float32))
    qg = rng.standard_normal((16, 512))
    kn = rng.standard_normal((2, 256))
    vn = rng.standard_normal((2, 256))
    O.gqa_append_kv_seq(kn[None], vn[None], p["k_norm_w"], kc, vc, O.BF16, start_pos=pos)
    out = O.gqa_attend_f64(qg, p["q_norm_w"], kc, vc, O.BF16, pos)
    # independent composition in numpy
    c, s = O.rope_tables(pos, prec=64)
    rot = lambda x: np.concatenate([x[:, :32] * c[:32] - x[:, 32:64] * s[:32],
                                    x[:, 32:64] * c[32:] + x[:, :32] * s[32:], x[:, 64:]], 1)
    nrm = lambda x, w: x / np.sqrt(np.mean(x * x, 1, keepdims=True) + 1e-6) * w
    kk = rot(nrm(kn, p["k_norm_w"]))
    assert np.array_equal(kc[pos], O.f32_to_bf16(kk.astype(np.float32)))
    assert np.array_equal(vc[pos], O.f32_to_bf16(vn.astype(np.float32)))
    q = rot(nrm(qg[:, :256], p["q_norm_w"]))
    K = O.bf16_to_f32(kc[:pos + 1]).astype(np.float64)
    V = O.bf16_to_f32(vc[:pos + 1]).astype(np.float64)
    ref = np_attention(q, K, V, 1 / 16) / (1 + np.exp(-qg[:, 256:]))
    assert np.allclose(out, ref, rtol=1e-10, atol=1e-12)
    # the fp32 reference-order path (half q, half output) stays within 2e-3
    out32 = O.gqa_attend(qg.astype(np.float32), p["q_norm_w"], kc, vc, O.BF16, pos)
    assert np.max(np.abs(out32 - ref)) < 2e-3


# ------------------------------------------------------------------ Q4
def np_unpack(w):
    """Independent unpack: element c = nibble (c % 8) of word c // 8."""
    rows, c8 = w.shape
    shifts = (np.arange(8, dtype=np.uint32) * 4)[None, None, :]
    return ((w[:, :, None] >> shifts) & 0xF).reshape(rows, c8 * 8)


def test_q4_nibble_order_kat():
    w = np.array([[0x76543210, 0xFEDCBA98] * 4], np.uint32)           # one 64-col group
    ones = np.array([[0x3C00]], np.uint16)                             # f16 1.0
    zeros = np.array([[0]], np.uint16)
    out = O.q4_dequant(w, ones, zeros, O.F16)
    assert out[0].tolist() == list(range(16)) * 4


@pytest.mark.parametrize("sb", ["f16", "bf16"])
def test_q4_dequant_closed_form_bit_exact(sb):
    w, s, b = synth.q4_weight(16, 256, seed=5, sb_dtype=sb)
    code = O.F16 if sb == "f16" else O.BF16
    out = O.q4_dequant(w, s, b, code)
    sf = np.repeat(O.to_real(s, code), 64, axis=1)
    bf = np.repeat(O.to_real(b, code), 64, axis=1)
    ref = (np_unpack(w).astype(np.float32) * sf + bf).astype(np.float32)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    # same values through an fp64 product rounded once: nibble*scale is exact
    ref64 = (np_unpack(w) * sf.astype(np.float64) + bf.astype(np.float64)).astype(np.float32)
    assert np.array_equal(out, ref64)
    # all-zero words give the bias, all-0xF words give 15*scale + bias
    z = O.q4_dequant(np.zeros_like(w), s, b, code)
    assert np.array_equal(z, bf)
    f = O.q4_dequant(np.full_like(w, 0xFFFFFFFF), s, b, code)
    assert np.array_equal(f, (np.float32(15) * sf + bf).astype(np.float32))


def test_q4_matvec_matches_dense_fp64(rng):
    w, s, b = synth.q4_weight(64, 2048, seed=7)
    x = rng.standard_normal(2048).astype(np.float32)
    dense = O.q4_dequant(w, s, b, O.F16).astype(np.float64)
    ref = dense @ x.astype(np.float64)
    y32 = O.q4_matvec(w, s, b, x)
    y64 = O.q4_matvec(w, s, b, x, prec=64)
    assert np.allclose(y64, ref, rtol=1e-12, atol=1e-12)
    assert np.max(np.abs(y32 - ref)) < 1e-4
