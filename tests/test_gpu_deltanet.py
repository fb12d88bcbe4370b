"""GPU parity of the DeltaNet entry points (qff_deltanet_decode / _prefill)
against the fp32 reference-order oracle (QwenDeltaNetKernel.swift:39-151 fed
token by token, QwenQ4ActiveExpertStreamingRunner.swift:1545-1561).

Tolerances (stated by the workload): outputs max-abs <= 2e-2 (bf16 outputs
may also be one bf16 ulp off where that exceeds 2e-2), fp32 state per-head
Frobenius relative error <= 1e-4. The conv state only shifts stored values,
so it must match bit for bit."""
import numpy as np
import pytest
import torch

from gpu_util import (DEV, assert_bf16_output_close, assert_f32_output_close, bf16_tensor,
                      f32_tensor, state_rel_err, to_np)
from oracle import oracle as O
from qff import synth

pytestmark = pytest.mark.gpu


def _params_gpu(p):
    return {k: f32_tensor(v) for k, v in p.items()}


def _oracle_decode(p, inp, in_f32=False):
    B = inp["qkv"].shape[0]
    outs, convs, ssms = [], [], []
    for s in range(B):
        qkv = inp["qkv_f32"][s] if in_f32 else O.bf16_to_f32(inp["qkv"][s])
        z = inp["z_f32"][s] if in_f32 else O.bf16_to_f32(inp["z"][s])
        o, c, st = O.deltanet_sequence(qkv[None], z[None], inp["a"][s][None], inp["b"][s][None],
                                       p["a_log"], p["dt_bias"], p["conv_w"], p["norm_w"],
                                       inp["conv_state"][s], inp["ssm_state"][s])
        outs.append(o[0]); convs.append(c); ssms.append(st)
    return np.stack(outs), np.stack(convs), np.stack(ssms)


@pytest.mark.parametrize("B", [1, 3, 16, 20, 32])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_deltanet_decode_matches_oracle(hip, B, out_dtype):
    import qff
    print(f"deltanet_decode B={B} out={out_dtype}", flush=True)
    p = synth.deltanet_params()
    inp = synth.deltanet_decode_inputs(B, seed=100 + B)
    ref_o, ref_c, ref_s = _oracle_decode(p, inp)
    ctx = qff.Context(max_batch=32, max_prefill_tokens=1)
    conv = f32_tensor(inp["conv_state"])
    ssm = f32_tensor(inp["ssm_state"])
    out = qff.deltanet_decode(ctx, _params_gpu(p), bf16_tensor(inp["qkv"]), bf16_tensor(inp["z"]),
                              f32_tensor(inp["a"]), f32_tensor(inp["b"]), conv, ssm,
                              out_dtype=out_dtype)
    torch.cuda.synchronize()
    if out_dtype == torch.bfloat16:
        assert_bf16_output_close(to_np(out), ref_o)
    else:
        assert_f32_output_close(to_np(out), ref_o)
    assert np.array_equal(to_np(conv), ref_c)
    assert state_rel_err(to_np(ssm), ref_s) <= 1e-4


@pytest.mark.parametrize("B", [4, 6])
def test_deltanet_decode_f32_inputs_and_repeat(hip, B):
    """fp32 activations, and three steps in a row on the same context and
    state buffers."""
    import qff
    p = synth.deltanet_params()
    inp = synth.deltanet_decode_inputs(B, seed=7)
    ctx = qff.Context(max_batch=8, max_prefill_tokens=1)
    conv = f32_tensor(inp["conv_state"])
    ssm = f32_tensor(inp["ssm_state"])
    pg = _params_gpu(p)
    rng = np.random.default_rng(8)
    for step in range(3):
        inp["qkv_f32"] = rng.standard_normal((B, 8192)).astype(np.float32)
        inp["z_f32"] = rng.standard_normal((B, 4096)).astype(np.float32)
        inp["a"] = rng.standard_normal((B, 32)).astype(np.float32)
        inp["b"] = rng.standard_normal((B, 32)).astype(np.float32)
        ref_o, ref_c, ref_s = _oracle_decode(p, inp, in_f32=True)
        out = qff.deltanet_decode(ctx, pg, f32_tensor(inp["qkv_f32"]), f32_tensor(inp["z_f32"]),
                                  f32_tensor(inp["a"]), f32_tensor(inp["b"]), conv, ssm,
                                  out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert_f32_output_close(to_np(out), ref_o)
        assert np.array_equal(to_np(conv), ref_c)
        assert state_rel_err(to_np(ssm), ref_s) <= 1e-4
        inp["conv_state"], inp["ssm_state"] = ref_c, ref_s


@pytest.mark.parametrize("T", [1, 3, 64, 130, 192, 200])
def test_deltanet_prefill_matches_sequential_oracle(hip, T):
    import qff
    print(f"deltanet_prefill T={T}", flush=True)
    p = synth.deltanet_params()
    inp = synth.deltanet_prefill_inputs(T, seed=300 + T)
    rng = np.random.default_rng(T)
    # a non-zero starting state exercises the conv history and state carry-in
    inp["conv_state"][:, 1:] = rng.standard_normal((8192, 3)).astype(np.float32)
    inp["ssm_state"] = (rng.standard_normal((32, 128, 128)) * 0.02).astype(np.float32)
    ref_o, ref_c, ref_s = O.deltanet_sequence(O.bf16_to_f32(inp["qkv"]), O.bf16_to_f32(inp["z"]),
                                              inp["a"], inp["b"], p["a_log"], p["dt_bias"],
                                              p["conv_w"], p["norm_w"], inp["conv_state"],
                                              inp["ssm_state"])
    ctx = qff.Context(max_batch=1, max_prefill_tokens=256)
    conv = f32_tensor(inp["conv_state"])
    ssm = f32_tensor(inp["ssm_state"])
    out = qff.deltanet_prefill(ctx, _params_gpu(p), bf16_tensor(inp["qkv"]), bf16_tensor(inp["z"]),
                               f32_tensor(inp["a"]), f32_tensor(inp["b"]), conv, ssm)
    torch.cuda.synchronize()
    assert_bf16_output_close(to_np(out), ref_o)
    assert np.array_equal(to_np(conv), ref_c)
    assert state_rel_err(to_np(ssm), ref_s) <= 1e-4


def _prefill_vs_oracle(p, inp, T, max_tokens=256):
    import qff
    ref_o, ref_c, ref_s = O.deltanet_sequence(O.bf16_to_f32(inp["qkv"]), O.bf16_to_f32(inp["z"]),
                                              inp["a"], inp["b"], p["a_log"], p["dt_bias"],
                                              p["conv_w"], p["norm_w"], inp["conv_state"],
                                              inp["ssm_state"])
    ctx = qff.Context(max_batch=1, max_prefill_tokens=max_tokens)
    conv = f32_tensor(inp["conv_state"])
    ssm = f32_tensor(inp["ssm_state"])
    out = qff.deltanet_prefill(ctx, _params_gpu(p), bf16_tensor(inp["qkv"]), bf16_tensor(inp["z"]),
                               f32_tensor(inp["a"]), f32_tensor(inp["b"]), conv, ssm,
                               out_dtype=torch.float32)
    torch.cuda.synchronize()
    return to_np(out), ref_o, to_np(conv), ref_c, to_np(ssm), ref_s


def _row_rel_err(got, ref, T):
    """Error of every (token, value head) row over that row's RMS."""
    g3, r3 = got.reshape(T, 32, 128).astype(np.float64), ref.reshape(T, 32, 128).astype(np.float64)
    rms = np.sqrt(np.mean(r3 ** 2, axis=2))
    return np.max(np.abs(g3 - r3), axis=2) / (rms + 1e-300)


@pytest.mark.parametrize("vscale", [2.0 ** -12, 2.0 ** 20])
def test_deltanet_prefill_value_scales(hip, vscale):
    """v channels scaled by 2^-12 and by 2^20 (q, k and the gates unchanged),
    from zero state, against the same inputs at scale 1: the output rows are
    formed and normalised in fp32-class arithmetic whose error is relative to
    the operands, so each row's error over its own RMS is no worse at either
    scale than at scale 1 (an fp16 intermediate would lose relative precision
    among its subnormals at 2^-12 and overflow at 2^20). The worst rows at
    every scale are those whose size comes from a nearly cancelled q.k (the
    Gram product's error is relative to |q||k|, ~1e-3 of the row there)."""
    T = 200
    print(f"deltanet_prefill v scale {vscale}", flush=True)
    p = synth.deltanet_params()
    base = synth.deltanet_prefill_inputs(T, seed=777)
    got1, ref1, _, _, _, _ = _prefill_vs_oracle(p, base, T)
    inp = {k: v.copy() for k, v in base.items()}
    v = O.bf16_to_f32(inp["qkv"][:, 4096:]) * np.float32(vscale)
    inp["qkv"][:, 4096:] = O.f32_to_bf16(v)
    got, ref, conv, ref_c, ssm, ref_s = _prefill_vs_oracle(p, inp, T)
    assert np.all(np.isfinite(got))
    assert_f32_output_close(got, ref)
    e1, es = _row_rel_err(got1, ref1, T), _row_rel_err(got, ref, T)
    print(f"row errors / RMS: scale 1 median {np.median(e1):.3g} max {e1.max():.3g}; "
          f"scale {vscale} median {np.median(es):.3g} max {es.max():.3g}", flush=True)
    assert np.median(es) <= 2 * np.median(e1) + 1e-6
    assert es.max() <= 2 * e1.max() + 1e-5
    assert np.array_equal(conv, ref_c)
    assert state_rel_err(ssm, ref_s) <= 1e-4


def test_deltanet_prefill_first_token_q_nearly_orthogonal_to_k(hip):
    """T = 1 from zero state with q nearly orthogonal to k in every key head:
    the output is beta (q.k) v / sqrt(128), with q.k ~ 1e-4 of |q||k|, so the
    pre-norm rows are four orders of magnitude below their usual size."""
    T = 1
    p = synth.deltanet_params()
    inp = synth.deltanet_prefill_inputs(T, seed=778)
    x = O.bf16_to_f32(inp["qkv"]).copy()
    w3 = p["conv_w"][:, 3]
    for kh in range(16):
        q0, k0 = kh * 128, 2048 + kh * 128
        # k = silu(w3 x) along key 127 only; q has a tiny component there
        x[0, k0:k0 + 127] = 0.0
        x[0, k0 + 127] = 2.0 / w3[k0 + 127]
        x[0, q0 + 127] = 1e-3 / w3[q0 + 127]
    inp["qkv"] = O.f32_to_bf16(x)
    got, ref, conv, ref_c, ssm, ref_s = _prefill_vs_oracle(p, inp, T)
    assert np.all(np.isfinite(got))
    assert_f32_output_close(got, ref)
    assert np.array_equal(conv, ref_c)
    assert state_rel_err(ssm, ref_s) <= 1e-4


def test_deltanet_prefill_config1_full_length(hip):
    """Config 1 at its full size: T = 4096 from zero state, against the
    4096-step sequential fp32 oracle (a few seconds of CPU)."""
    import qff
    p = synth.deltanet_params()
    inp = synth.deltanet_prefill_inputs(4096)
    print("deltanet_prefill T=4096 (oracle running)", flush=True)
    ref_o, ref_c, ref_s = O.deltanet_sequence(O.bf16_to_f32(inp["qkv"]), O.bf16_to_f32(inp["z"]),
                                              inp["a"], inp["b"], p["a_log"], p["dt_bias"],
                                              p["conv_w"], p["norm_w"], inp["conv_state"],
                                              inp["ssm_state"])
    ctx = qff.Context(max_batch=1, max_prefill_tokens=4096)
    conv = f32_tensor(inp["conv_state"])
    ssm = f32_tensor(inp["ssm_state"])
    out = qff.deltanet_prefill(ctx, _params_gpu(p), bf16_tensor(inp["qkv"]), bf16_tensor(inp["z"]),
                               f32_tensor(inp["a"]), f32_tensor(inp["b"]), conv, ssm)
    torch.cuda.synchronize()
    assert_bf16_output_close(to_np(out), ref_o)
    assert np.array_equal(to_np(conv), ref_c)
    assert state_rel_err(to_np(ssm), ref_s) <= 1e-4


def test_deltanet_rejects_bad_arguments(hip):
    import qff
    p = _params_gpu(synth.deltanet_params())
    ctx = qff.Context(max_batch=2, max_prefill_tokens=16)
    x = torch.zeros(4, 8192, dtype=torch.bfloat16, device=DEV)
    z = torch.zeros(4, 4096, dtype=torch.bfloat16, device=DEV)
    ab = torch.zeros(4, 32, device=DEV)
    conv = torch.zeros(4, 8192, 4, device=DEV)
    ssm = torch.zeros(4, 32, 128, 128, device=DEV)
    with pytest.raises(qff.QffError) as e:           # batch above the context's max
        qff.deltanet_decode(ctx, p, x, z, ab, ab, conv, ssm)
    assert e.value.status == -4
    with pytest.raises(qff.QffError) as e:           # chunk other than 64
        qff.deltanet_prefill(ctx, p, x, z, ab, ab, conv[0], ssm[0], chunk=32)
    assert e.value.status == -2
    with pytest.raises(qff.QffError) as e:           # T above max_prefill_tokens
        qff.deltanet_prefill(ctx, p, torch.zeros(17, 8192, dtype=torch.bfloat16, device=DEV),
                             torch.zeros(17, 4096, dtype=torch.bfloat16, device=DEV),
                             torch.zeros(17, 32, device=DEV), torch.zeros(17, 32, device=DEV),
                             conv[0], ssm[0])
    assert e.value.status == -4


@pytest.mark.parametrize("B,T", [(1, 4096), (6, 1024)])
def test_deltanet_decode_consecutive_steps(hip, B, T):
    """qff_deltanet_decode, the reference's per-token path
    (QwenQ4ActiveExpertStreamingRunner.swift:1545-1561 -> deltanet.metal
    :250-356), T steps in a row on the config-1 inputs from zero state (batch
    1: 4096 steps; batch 6: 1024 steps of six independent sequences),
    against the sequential fp32 oracle: every step's output within the bf16
    bar and the state rel <= 1e-4 at the end."""
    import qff
    print(f"deltanet_decode {T} consecutive steps B={B} (oracle running)", flush=True)
    p = synth.deltanet_params()
    seqs = [synth.deltanet_prefill_inputs(T, seed=900 + s) for s in range(B)]
    refs = [O.deltanet_sequence(O.bf16_to_f32(inp["qkv"]), O.bf16_to_f32(inp["z"]), inp["a"], inp["b"],
                                p["a_log"], p["dt_bias"], p["conv_w"], p["norm_w"], inp["conv_state"],
                                inp["ssm_state"]) for inp in seqs]
    # token-major across the batch: step t feeds row t of every sequence
    qkv = bf16_tensor(np.stack([s["qkv"] for s in seqs], 1))       # [T, B, 8192]
    z = bf16_tensor(np.stack([s["z"] for s in seqs], 1))
    a = f32_tensor(np.stack([s["a"] for s in seqs], 1))
    b = f32_tensor(np.stack([s["b"] for s in seqs], 1))
    ctx = qff.Context(max_batch=8, max_prefill_tokens=1)
    conv = torch.zeros(B, 8192, 4, device=DEV)
    ssm = torch.zeros(B, 32, 128, 128, device=DEV)
    out = torch.empty(T, B, 4096, dtype=torch.bfloat16, device=DEV)
    pg = _params_gpu(p)
    print("  GPU steps", flush=True)
    for t in range(T):
        qff.deltanet_decode(ctx, pg, qkv[t], z[t], a[t], b[t], conv, ssm, out=out[t])
    torch.cuda.synchronize()
    got = to_np(out)
    for s in range(B):
        ref_o, ref_c, ref_s = refs[s]
        assert_bf16_output_close(got[:, s], ref_o)
        assert np.array_equal(to_np(conv)[s], ref_c)
        rel = state_rel_err(to_np(ssm)[s], ref_s)
        print(f"  seq {s}: state rel {rel:.3g}", flush=True)
        assert rel <= 1e-4


@pytest.mark.parametrize("T", [70, 200])
def test_deltanet_prefill_f32_inputs(hip, T):
    """fp32 qkv / z (in_dtype F32) through the chunked prefill from a
    non-zero state, fp32 and bf16 outputs, against the oracle fed the same
    fp32 values."""
    import qff
    print(f"deltanet_prefill f32 inputs T={T}", flush=True)
    p = synth.deltanet_params()
    rng = np.random.default_rng(600 + T)
    qkv = rng.standard_normal((T, 8192)).astype(np.float32)
    z = rng.standard_normal((T, 4096)).astype(np.float32)
    a = rng.standard_normal((T, 32)).astype(np.float32)
    b = rng.standard_normal((T, 32)).astype(np.float32)
    conv0 = np.zeros((8192, 4), np.float32)
    conv0[:, 1:] = rng.standard_normal((8192, 3)).astype(np.float32)
    ssm0 = (rng.standard_normal((32, 128, 128)) * 0.02).astype(np.float32)
    ref_o, ref_c, ref_s = O.deltanet_sequence(qkv, z, a, b, p["a_log"], p["dt_bias"], p["conv_w"], p["norm_w"],
                                              conv0, ssm0)
    ctx = qff.Context(max_batch=1, max_prefill_tokens=256)
    for out_dtype in (torch.float32, torch.bfloat16):
        conv, ssm = f32_tensor(conv0), f32_tensor(ssm0)
        out = qff.deltanet_prefill(ctx, _params_gpu(p), f32_tensor(qkv), f32_tensor(z), f32_tensor(a),
                                   f32_tensor(b), conv, ssm, out_dtype=out_dtype)
        torch.cuda.synchronize()
        if out_dtype == torch.float32:
            assert_f32_output_close(to_np(out), ref_o)
        else:
            assert_bf16_output_close(to_np(out), ref_o)
        assert np.array_equal(to_np(conv), ref_c)
        assert state_rel_err(to_np(ssm), ref_s) <= 1e-4


def test_deltanet_prefill_graph_replay(hip):
    """The chunk-local pass takes its (chunk, key head) units from a work-queue
    counter in the context that each launch's last workgroup resets. A
    captured prefill (T = 200, four chunks with a ragged tail) is replayed
    three times, each replay continuing from the conv state and state the
    previous one left, with an eager prefill of another length on the same
    context between replays: every replay's output, conv state and state
    against the sequential oracle."""
    import qff
    p = synth.deltanet_params()
    pg = _params_gpu(p)
    ctx = qff.Context(max_batch=1, max_prefill_tokens=256)
    T = 200
    inp = synth.deltanet_prefill_inputs(T, seed=900)
    qkv, z = bf16_tensor(inp["qkv"]), bf16_tensor(inp["z"])
    a, b = f32_tensor(inp["a"]), f32_tensor(inp["b"])
    conv = f32_tensor(inp["conv_state"])
    ssm = f32_tensor(inp["ssm_state"])
    out = torch.empty(T, 4096, dtype=torch.bfloat16, device=DEV)
    other = synth.deltanet_prefill_inputs(70, seed=901)
    o_args = [bf16_tensor(other["qkv"]), bf16_tensor(other["z"]), f32_tensor(other["a"]), f32_tensor(other["b"])]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        # warm-up call outside the graph, on scratch copies of the state
        qff.deltanet_prefill(ctx, pg, qkv, z, a, b, conv.clone(), ssm.clone(), out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    print(f"deltanet_prefill graph capture T={T}", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        qff.deltanet_prefill(ctx, pg, qkv, z, a, b, conv, ssm, out=out)
    x, zz = O.bf16_to_f32(inp["qkv"]), O.bf16_to_f32(inp["z"])
    cs, ss = inp["conv_state"], inp["ssm_state"]
    for rep in range(3):
        print(f"deltanet_prefill graph replay {rep}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        ref_o, cs, ss = O.deltanet_sequence(x, zz, inp["a"], inp["b"], p["a_log"], p["dt_bias"], p["conv_w"],
                                            p["norm_w"], cs, ss)
        assert_bf16_output_close(to_np(out), ref_o)
        assert np.array_equal(to_np(conv), cs), f"replay {rep}: conv state"
        assert state_rel_err(to_np(ssm), ss) <= 1e-4, f"replay {rep}"
        # an eager prefill of another length on the same context
        qff.deltanet_prefill(ctx, pg, *o_args, f32_tensor(other["conv_state"]), f32_tensor(other["ssm_state"]))
        torch.cuda.synchronize()


def test_deltanet_decode_batches_alternate_and_graph_replay(hip):
    """The two value heads of a key head share its q/k conv-state slots; the
    second workgroup to finish reading them rewrites them, counted on
    per-(sequence, key head) counters in the context that every launch
    leaves at zero. Calls of different batch sizes on one context, then a
    captured step replayed three times (eager work and a sync between the
    replays): every output, conv state and state against the oracle."""
    import qff
    p = synth.deltanet_params()
    pg = _params_gpu(p)
    ctx = qff.Context(max_batch=32, max_prefill_tokens=1)
    for B in (32, 2, 17, 1, 32):
        print(f"deltanet_decode alternate B={B}", flush=True)
        inp = synth.deltanet_decode_inputs(B, seed=300 + B)
        ref_o, ref_c, ref_s = _oracle_decode(p, inp)
        conv = f32_tensor(inp["conv_state"])
        ssm = f32_tensor(inp["ssm_state"])
        out = qff.deltanet_decode(ctx, pg, bf16_tensor(inp["qkv"]), bf16_tensor(inp["z"]), f32_tensor(inp["a"]),
                                  f32_tensor(inp["b"]), conv, ssm, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert_f32_output_close(to_np(out), ref_o)
        assert np.array_equal(to_np(conv), ref_c)
        assert state_rel_err(to_np(ssm), ref_s) <= 1e-4

    B = 5
    print(f"deltanet_decode graph replay B={B}", flush=True)
    inp = synth.deltanet_decode_inputs(B, seed=77)
    qkv, z = bf16_tensor(inp["qkv"]), bf16_tensor(inp["z"])
    a, b = f32_tensor(inp["a"]), f32_tensor(inp["b"])
    conv = f32_tensor(inp["conv_state"])
    ssm = f32_tensor(inp["ssm_state"])
    out = torch.empty(B, 4096, dtype=torch.float32, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        # warm-up call outside the graph, on scratch copies of the state
        c2, s2 = conv.clone(), ssm.clone()
        qff.deltanet_decode(ctx, pg, qkv, z, a, b, c2, s2, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        qff.deltanet_decode(ctx, pg, qkv, z, a, b, conv, ssm, out=out)
    cs, ss = inp["conv_state"], inp["ssm_state"]
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        inp["conv_state"], inp["ssm_state"] = cs, ss
        ref_o, cs, ss = _oracle_decode(p, inp)
        assert_f32_output_close(to_np(out), ref_o)
        assert np.array_equal(to_np(conv), cs), f"replay {rep}: conv state"
        assert state_rel_err(to_np(ssm), ss) <= 1e-4, f"replay {rep}"
        # eager work between replays on the same context
        c2, s2 = conv.clone(), ssm.clone()
        qff.deltanet_decode(ctx, pg, qkv, z, a, b, c2, s2)
        torch.cuda.synchronize()
