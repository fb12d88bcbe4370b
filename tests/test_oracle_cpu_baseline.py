"""The timed CPU baselines of the full-attention prefill and of the config-4
layers (oracle/cpu_baseline.c: qffb_gqa_prefill_tokens, qffb_dn_layer_decode,
qffb_gqa_layer_decode) reproduce the oracle's own composition of the same
fp32 functions bit for bit (fp32 caches and no fp16 rounding of q or of the
attention output on both sides, which is how the baselines are built), so
the baseline times the reference's algorithm and nothing else."""
import numpy as np
import pytest

from oracle import cpu_baseline as CB
from oracle import oracle as O
from qff import synth


def _q4(rows, cols, seed):
    w, s, b = synth.q4_weight(rows, cols, seed=seed)
    return w, O.f16_to_f32(s), O.f16_to_f32(b), (w, s, b)


def _eq(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("threads", [1, 3])
def test_gqa_prefill_tokens_equals_oracle(threads):
    T, H = 21, 2048
    rng = np.random.default_rng(40)
    x = rng.standard_normal((T, H)).astype(np.float32)
    parts = [_q4(r, H, 400 + i) for i, r in enumerate((8192, 512, 512))]
    w, sc, bi = CB.q4_stack([p[:3] for p in parts])
    gp = synth.gqa_params()
    K = np.zeros((T, 2, 256), np.float32)
    V = np.zeros_like(K)
    out = np.zeros((T, 16, 256), np.float32)
    CB.gqa_prefill_tokens(CB.load(), 0, T, x, w, sc, bi, gp["q_norm_w"], gp["k_norm_w"], K, V, out, threads=threads)
    kc = np.zeros((T, 2, 256), np.float32)
    vc = np.zeros_like(kc)
    for t in range(T):
        qg, k, v = (O.q4_matvec(*p[3], x[t]) for p in parts)
        O.gqa_append_kv_seq(k.reshape(1, 2, 256), v.reshape(1, 2, 256), gp["k_norm_w"], kc, vc, O.F32,
                            start_pos=t)
        ref = O.gqa_attend(qg.reshape(16, 512), gp["q_norm_w"], kc, vc, O.F32, t, q_dtype=O.F32, attn_dtype=O.F32)
        assert _eq(out[t], ref), f"token {t}"
    assert _eq(K, kc) and _eq(V, vc)


def test_layer_decode_equals_oracle():
    """One DeltaNet and one full-attention attention block at batch 2."""
    B, H = 2, 2048
    rng = np.random.default_rng(41)
    L = CB.load()
    p = synth.deltanet_params()
    norm_w = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    dn_in = [_q4(r, H, 410 + i) for i, r in enumerate((8192, 4096, 32, 32))]
    dn_out = _q4(2048, 4096, 415)
    x = rng.standard_normal((B, H)).astype(np.float32)
    conv = rng.standard_normal((B, 8192, 4)).astype(np.float32)
    ssm = (rng.standard_normal((B, 32, 128, 128)) * 0.02).astype(np.float32)
    xg, cg, sg = x.copy(), conv.copy(), ssm.copy()
    CB.dn_layer_decode(L, xg, norm_w, CB.q4_stack([q[:3] for q in dn_in]), CB.q4_stack([dn_out[:3]]), p, cg, sg,
                       threads=2)
    for s in range(B):
        xn = O.rmsnorm(x[s], norm_w)
        qkv, z, bb, aa = (O.q4_matvec(*q[3], xn) for q in dn_in)
        o, cs, ss = O.deltanet_sequence(qkv[None], z[None], aa[None], bb[None], p["a_log"], p["dt_bias"],
                                        p["conv_w"], p["norm_w"], conv[s], ssm[s])
        assert _eq(xg[s], x[s] + O.q4_matvec(*dn_out[3], o[0]))
        assert _eq(cg[s], cs) and _eq(sg[s], ss)
    gp = synth.gqa_params()
    g_in = [_q4(r, H, 420 + i) for i, r in enumerate((8192, 512, 512))]
    g_out = _q4(2048, 4096, 425)
    max_ctx = 50
    K = rng.standard_normal((B, max_ctx, 2, 256)).astype(np.float32)
    V = rng.standard_normal((B, max_ctx, 2, 256)).astype(np.float32)
    pos = np.array([7, 49], np.int32)
    xg, Kg, Vg = x.copy(), K.copy(), V.copy()
    CB.gqa_layer_decode(L, xg, norm_w, CB.q4_stack([q[:3] for q in g_in]), CB.q4_stack([g_out[:3]]),
                        gp["q_norm_w"], gp["k_norm_w"], Kg, Vg, pos, threads=2)
    for s in range(B):
        xn = O.rmsnorm(x[s], norm_w)
        qg, k, v = (O.q4_matvec(*q[3], xn) for q in g_in)
        kc, vc = K[s].copy(), V[s].copy()
        O.gqa_append_kv_seq(k.reshape(1, 2, 256), v.reshape(1, 2, 256), gp["k_norm_w"], kc, vc, O.F32,
                            start_pos=int(pos[s]))
        att = O.gqa_attend(qg.reshape(16, 512), gp["q_norm_w"], kc, vc, O.F32, int(pos[s]), q_dtype=O.F32,
                           attn_dtype=O.F32)
        assert _eq(xg[s], x[s] + O.q4_matvec(*g_out[3], att.reshape(4096)))
        assert _eq(Kg[s], kc) and _eq(Vg[s], vc)
