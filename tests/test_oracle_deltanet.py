"""Pins the DeltaNet half of the oracle (QwenDeltaNetKernel.swift:4-256,
deltanet.metal:112-356) with closed forms, invariants, an independent matrix
formulation, and the chunked (WY / UT) identity the HIP prefill relies on."""
import numpy as np
import pytest

from oracle import oracle as O
from qff import synth


def np_silu(x):
    return x / (1.0 + np.exp(-x))


def np_softplus(x):
    return np.where(x > 20, x, np.where(x < -20, np.exp(x), np.log1p(np.exp(x))))


def test_scalar_activations():
    for x in (-30.0, -20.5, -3.0, 0.0, 0.7, 19.9, 20.5):
        assert abs(O.silu(x, 64) - x / (1 + np.exp(-x))) < 1e-12
        assert abs(O.sigmoid(x, 64) - 1 / (1 + np.exp(-x))) < 1e-12
        assert abs(O.softplus(x, 64) - float(np_softplus(np.float64(x)))) < 1e-12
    # clamps of QwenDeltaNetKernel.swift:16-19: identity above 20, exp below -20
    assert O.softplus(25.0) == 25.0
    assert O.softplus(-25.0) == np.float32(np.exp(np.float32(-25.0)))


def test_conv1d_identity_tap_and_shift(rng):
    dim = 64
    x = rng.standard_normal(dim).astype(np.float32)
    st = rng.standard_normal((dim, 4)).astype(np.float32)
    w = np.zeros((dim, 4), np.float32)
    w[:, 3] = 1.0                       # only the newest tap
    out, st2 = O.conv1d_step(x, st, w)
    assert np.array_equal(out, np.array([O.silu(float(v)) for v in x], np.float32))
    assert np.array_equal(st2[:, :3], st[:, 1:]) and np.array_equal(st2[:, 3], x)
    w = np.zeros((dim, 4), np.float32)
    w[:, 0] = 1.0                       # only the oldest tap = old slot 1
    out, _ = O.conv1d_step(x, st, w)
    assert np.allclose(out, np_silu(st[:, 1].astype(np.float64)), rtol=1e-6, atol=1e-7)


def test_conv1d_sequence_matches_causal_convolution(rng):
    T, dim = 12, 32
    xs = rng.standard_normal((T, dim))
    w = rng.standard_normal((dim, 4))
    st = np.zeros((dim, 4))
    for t in range(T):
        out, st = O.conv1d_step(xs[t], st, w, prec=64)
        # causal conv with zero padding: tap j multiplies x[t-3+j]
        ref = sum(w[:, j] * (xs[t - 3 + j] if t - 3 + j >= 0 else 0.0) for j in range(4))
        assert np.allclose(out, np_silu(ref), rtol=1e-12, atol=1e-14)


def test_l2norm_unit_norm(rng):
    v = rng.standard_normal(128).astype(np.float32)
    out = O.l2norm(v)
    assert abs(np.linalg.norm(out.astype(np.float64)) - 1.0) < 1e-6
    # eps enters inside the sqrt: a zero vector stays zero
    assert np.all(O.l2norm(np.zeros(128, np.float32)) == 0)


def _np_step(q, k, v, a, b, a_log, dt_bias, S):
    """Matrix form of one gated delta-rule step in fp64: S <- g S;
    S <- S + beta (v - S k) k^T; o = S q. Rows of S are v, columns k."""
    S = S.copy()
    out = np.zeros((32, 128))
    for h in range(32):
        beta = 1 / (1 + np.exp(-b[h]))
        g = np.exp(-np.exp(a_log[h]) * np_softplus(a[h] + dt_bias[h]))
        S[h] *= g
        S[h] += beta * np.outer(v[h] - S[h] @ k[h], k[h])
        out[h] = S[h] @ q[h]
    return out, S


def test_delta_rule_matches_matrix_form(rng):
    q, k, v = (rng.standard_normal((32, 128)) for _ in range(3))
    a, b, al, dtb = (rng.standard_normal(32) for _ in range(4))
    S = rng.standard_normal((32, 128, 128)) * 0.02
    out, S2 = O.deltanet_recurrent_step(q, k, v, a, b, al, dtb, S, prec=64)
    ref_o, ref_S = _np_step(q, k, v, a, b, al, dtb, S)
    assert np.allclose(S2, ref_S, rtol=1e-12, atol=1e-13)
    assert np.allclose(out, ref_o, rtol=1e-11, atol=1e-12)
    # a transposed state (rows = k) would not match: pin the orientation
    _, ref_T = _np_step(q, k, v, a, b, al, dtb, np.swapaxes(S, 1, 2))
    assert not np.allclose(S2, np.swapaxes(ref_T, 1, 2), atol=1e-6)


def test_delta_rule_beta_zero_is_pure_decay(rng):
    q, k, v = (rng.standard_normal((32, 128)).astype(np.float32) for _ in range(3))
    a, al, dtb = (rng.standard_normal(32).astype(np.float32) for _ in range(3))
    b = np.full(32, -200.0, np.float32)          # sigmoid(-200) == 0 in fp32
    S = (rng.standard_normal((32, 128, 128)) * 0.02).astype(np.float32)
    out, S2 = O.deltanet_recurrent_step(q, k, v, a, b, al, dtb, S)
    g = np.exp(-np.exp(al.astype(np.float64)) * np_softplus((a + dtb).astype(np.float64)))
    assert np.allclose(S2, S * g[:, None, None], rtol=2e-6, atol=1e-9)


def test_delta_rule_unit_gate_writes_value(rng):
    # g = 1 (A_log = -200 -> exp underflows to 0), beta = 1, |k| = 1:
    # the delta rule stores v under key k exactly: S' k = v
    q = rng.standard_normal((32, 128)).astype(np.float32)
    k = rng.standard_normal((32, 128))
    k = (k / np.linalg.norm(k, axis=1, keepdims=True)).astype(np.float32)
    v = rng.standard_normal((32, 128)).astype(np.float32)
    a = rng.standard_normal(32).astype(np.float32)
    b = np.full(32, 200.0, np.float32)
    al = np.full(32, -200.0, np.float32)
    dtb = np.zeros(32, np.float32)
    S = (rng.standard_normal((32, 128, 128)) * 0.02).astype(np.float32)
    _, S2 = O.deltanet_recurrent_step(q, k, v, a, b, al, dtb, S)
    Sk = np.einsum("hrc,hc->hr", S2.astype(np.float64), k.astype(np.float64))
    assert np.max(np.abs(Sk - v)) < 2e-5


def test_delta_rule_zero_state_single_step(rng):
    # from S = 0: S' = beta v k^T, so o = beta v (k . q)
    q, k, v = (rng.standard_normal((32, 128)) for _ in range(3))
    a, b, al, dtb = (rng.standard_normal(32) for _ in range(4))
    out, _ = O.deltanet_recurrent_step(q, k, v, a, b, al, dtb, np.zeros((32, 128, 128)), prec=64)
    beta = 1 / (1 + np.exp(-b))
    ref = beta[:, None] * v * np.sum(k * q, axis=1)[:, None]
    assert np.allclose(out, ref, rtol=1e-12, atol=1e-12)


def test_gated_rmsnorm_closed_form(rng):
    core = rng.standard_normal(4096)
    w = rng.standard_normal(128)
    z = rng.standard_normal(4096)
    out = O.gated_rmsnorm(core, w, z, prec=64)
    c = core.reshape(32, 128)
    inv = 1 / np.sqrt(np.mean(c * c, axis=1, keepdims=True) + 1e-6)
    ref = (c * inv * w[None, :] * np_silu(z.reshape(32, 128))).reshape(-1)
    assert np.allclose(out, ref, rtol=1e-12, atol=1e-14)
    assert np.all(O.gated_rmsnorm(core, w, np.zeros(4096), prec=64) == 0)


def np_layer_token(qkv, z, a, b, p, conv_state, S):
    """fp64 restatement of one token through the layer core in matrix form:
    conv + SiLU, q/k L2 norm (q / sqrt(128)), k-head h//2 feeds v-heads h."""
    conv_state = np.concatenate([conv_state[:, 1:], qkv[:, None]], axis=1)
    x = np_silu(np.sum(conv_state * p["conv_w"], axis=1))
    q = x[:2048].reshape(16, 128)
    k = x[2048:4096].reshape(16, 128)
    q = q / np.sqrt(np.sum(q * q, 1, keepdims=True) + 1e-6) / np.sqrt(128.0)
    k = k / np.sqrt(np.sum(k * k, 1, keepdims=True) + 1e-6)
    q, k = np.repeat(q, 2, axis=0), np.repeat(k, 2, axis=0)
    v = x[4096:].reshape(32, 128)
    o, S = _np_step(q, k, v, a, b, p["a_log"], p["dt_bias"], S)
    inv = 1 / np.sqrt(np.mean(o * o, axis=1, keepdims=True) + 1e-6)
    out = (o * inv * p["norm_w"][None, :] * np_silu(z.reshape(32, 128))).reshape(-1)
    return out, conv_state, S


def test_layer_sequence_matches_matrix_form():
    p = {k: v.astype(np.float64) for k, v in synth.deltanet_params().items()}
    inp = synth.deltanet_prefill_inputs(T=6)
    qkv = O.bf16_to_f32(inp["qkv"]).astype(np.float64)
    z = O.bf16_to_f32(inp["z"]).astype(np.float64)
    a, b = inp["a"].astype(np.float64), inp["b"].astype(np.float64)
    cs = np.random.default_rng(3).standard_normal((8192, 4))
    S = np.random.default_rng(4).standard_normal((32, 128, 128)) * 0.02
    out, cs2, S2 = O.deltanet_sequence(qkv, z, a, b, p["a_log"], p["dt_bias"], p["conv_w"],
                                       p["norm_w"], cs, S, prec=64)
    rc, rS = cs.copy(), S.copy()
    for t in range(6):
        ro, rc, rS = np_layer_token(qkv[t], z[t], a[t], b[t], p, rc, rS)
        assert np.allclose(out[t], ro, rtol=1e-10, atol=1e-11)
    assert np.allclose(S2, rS, rtol=1e-11, atol=1e-13)
    assert np.allclose(cs2, rc)


def test_fp32_reference_order_close_to_fp64():
    p = synth.deltanet_params()
    inp = synth.deltanet_prefill_inputs(T=32)
    qkv, z = O.bf16_to_f32(inp["qkv"]), O.bf16_to_f32(inp["z"])
    args = (inp["a"], inp["b"], p["a_log"], p["dt_bias"], p["conv_w"], p["norm_w"],
            inp["conv_state"], inp["ssm_state"])
    o32, _, s32 = O.deltanet_sequence(qkv, z, *args, prec=32)
    o64, _, s64 = O.deltanet_sequence(qkv, z, *args, prec=64)
    assert np.max(np.abs(o32 - o64)) < 1e-4
    rel = np.linalg.norm((s32 - s64).reshape(32, -1), axis=1) / np.linalg.norm(s64.reshape(32, -1), axis=1)
    assert rel.max() < 1e-5


# ----------------------------------------------------------------------------
# Chunked (WY / UT) form. Within a chunk with cumulative log gates G_i:
#   A_ij = beta_i exp(G_i - G_j) (k_i . k_j) for j < i,   T = (I + A)^-1
#   W = T (beta exp(G) K),  U~ = T (beta V),  U = U~ - W S0^T
#   O = (exp(G) Q) S0^T + (exp(G_i - G_j) [j <= i] * Q K^T) U
#   S_C = exp(G_C) S0 + U^T (exp(G_C - G) K)
# It is an identity of the sequential recurrence: the fp64 chunked form must
# reproduce the fp64 oracle to rounding. This pins the algebra the HIP
# chunked prefill implements.
def chunked_heads(q, k, v, beta, logg, S0, C):
    """q,k,v [T,H,d]; beta, logg [T,H]; S0 [H,d,d] rows=v. Returns o, S."""
    T, H, d = q.shape
    S = S0.copy()
    o = np.zeros((T, H, d))
    for h in range(H):
        for c0 in range(0, T, C):
            sl = slice(c0, min(T, c0 + C))
            Q, K, V = q[sl, h], k[sl, h], v[sl, h]
            bt, G = beta[sl, h], np.cumsum(logg[sl, h])
            n = len(G)
            D = np.exp(G[:, None] - G[None, :])
            A = np.tril(bt[:, None] * D * (K @ K.T), -1)
            Tm = np.linalg.inv(np.eye(n) + A)
            W = Tm @ (bt[:, None] * np.exp(G)[:, None] * K)
            U = Tm @ (bt[:, None] * V) - W @ S[h].T
            o[sl, h] = (np.exp(G)[:, None] * Q) @ S[h].T + (np.tril(D) * (Q @ K.T)) @ U
            S[h] = np.exp(G[-1]) * S[h] + U.T @ (np.exp(G[-1] - G)[:, None] * K)
    return o, S


@pytest.mark.parametrize("T,C", [(64, 64), (100, 32), (192, 64)])
def test_chunked_form_equals_sequential(T, C):
    rng = np.random.default_rng(T + C)
    H, d = 4, 128
    q = rng.standard_normal((T, H, d))
    k = rng.standard_normal((T, H, d))
    k /= np.linalg.norm(k, axis=2, keepdims=True)
    q /= np.linalg.norm(q, axis=2, keepdims=True) * np.sqrt(d)
    v = rng.standard_normal((T, H, d))
    b = rng.standard_normal((T, H))
    a = rng.standard_normal((T, H))
    al = rng.uniform(-1, 1, H)
    dtb = rng.standard_normal(H) * 0.1
    beta = 1 / (1 + np.exp(-b))
    logg = -np.exp(al)[None, :] * np_softplus(a + dtb[None, :])
    S0 = rng.standard_normal((H, d, d)) * 0.02
    oc, Sc = chunked_heads(q, k, v, beta, logg, S0, C)
    # sequential oracle over the same heads (pad to its 32-head layout)
    S = np.zeros((32, d, d)); S[:H] = S0
    for t in range(T):
        qq = np.zeros((32, d)); kk = np.zeros((32, d)); vv = np.zeros((32, d))
        qq[:H], kk[:H], vv[:H] = q[t], k[t], v[t]
        aa = np.zeros(32); bb = np.zeros(32); AL = np.zeros(32); DT = np.zeros(32)
        aa[:H], bb[:H], AL[:H], DT[:H] = a[t], b[t], al, dtb
        out, S = O.deltanet_recurrent_step(qq, kk, vv, aa, bb, AL, DT, S, prec=64)
        assert np.allclose(out[:H], oc[t], rtol=1e-9, atol=1e-12)
    assert np.allclose(S[:H], Sc, rtol=1e-9, atol=1e-13)


@pytest.mark.parametrize("threads", [1, 4])
def test_cpu_baseline_equals_oracle_bit_for_bit(threads):
    """The timed CPU baseline (oracle/cpu_baseline.c: the same fp32 functions,
    independent channels / heads spread over OpenMP threads) reproduces the
    sequential oracle exactly, from a non-zero state."""
    from oracle import cpu_baseline as CB
    p = synth.deltanet_params()
    inp = synth.deltanet_prefill_inputs(37, seed=5)
    rng = np.random.default_rng(6)
    inp["conv_state"][:, 1:] = rng.standard_normal((8192, 3)).astype(np.float32)
    inp["ssm_state"] = (rng.standard_normal((32, 128, 128)) * 0.02).astype(np.float32)
    qkv, z = O.bf16_to_f32(inp["qkv"]), O.bf16_to_f32(inp["z"])
    ref = O.deltanet_sequence(qkv, z, inp["a"], inp["b"], p["a_log"], p["dt_bias"], p["conv_w"], p["norm_w"],
                              inp["conv_state"], inp["ssm_state"])
    got = CB.deltanet_prefill(CB.load(), qkv, z, inp["a"], inp["b"], p, inp["conv_state"], inp["ssm_state"],
                              threads=threads)
    for g, r in zip(got, ref):
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32))


def test_cpu_baseline_attention_equals_oracle():
    """The baseline's batched split-KV attention equals the oracle's per
    sequence bit for bit (reference geometry NC = min(16, L))."""
    from oracle import cpu_baseline as CB
    rng = np.random.default_rng(9)
    B, max_ctx = 3, 300
    lengths = np.array([1, 17, 300], np.int32)
    q = rng.standard_normal((B, 16, 256)).astype(np.float32)
    K = rng.standard_normal((B, max_ctx, 2, 256)).astype(np.float32)
    V = rng.standard_normal((B, max_ctx, 2, 256)).astype(np.float32)
    got = CB.attention_decode(CB.load(), q, K, V, lengths, threads=2)
    for s in range(B):
        ref = O.attention_decode(q[s], K[s, :lengths[s]], V[s, :lengths[s]])
        assert np.array_equal(got[s].view(np.uint32), ref.view(np.uint32))
