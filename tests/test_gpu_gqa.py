"""GPU parity of qff_gqa_decode against the fp32 reference-order oracle
(deltanet.metal:599-708, attention.metal:134-377, Attention.swift:129-157,
QwenQ4ActiveExpertStreamingRunner.swift:1076-1150, with the reference's
half rounding of q and of the attention output).

Tolerance: outputs max-abs <= 2e-2 (bf16 outputs may also be one bf16 ulp
off where that exceeds 2e-2). The appended cache entries are the bf16
rounding of fp32 values that the two sides compute in a different order, so
they must agree to one bf16 ulp; every other cache entry must be untouched."""
import numpy as np
import pytest
import torch

from gpu_util import (DEV, assert_bf16_output_close, assert_f32_output_close, bf16_tensor,
                      bf16_ulp, f32_tensor, to_np)
from oracle import oracle as O
from qff import synth

pytestmark = pytest.mark.gpu


def _run_case(hip, lengths, max_ctx, out_dtype=torch.float32, seed=11):
    import qff
    B = len(lengths)
    print(f"gqa_decode B={B} max_ctx={max_ctx} lengths={list(lengths)[:8]}", flush=True)
    p = synth.gqa_params()
    inp = synth.gqa_decode_inputs(B, max_ctx, seed=seed, lengths=lengths)
    ctx = qff.Context(max_batch=max(B, 1), max_ctx=max_ctx, max_prefill_tokens=1)
    kc = bf16_tensor(inp["k_cache"])
    vc = bf16_tensor(inp["v_cache"])
    pg = {k: f32_tensor(v) for k, v in p.items()}
    pos_t = torch.from_numpy(inp["positions"]).to(DEV)
    out = qff.gqa_decode(ctx, pg, bf16_tensor(inp["q_gate"]), bf16_tensor(inp["k_new"]),
                         bf16_tensor(inp["v_new"]), kc, vc, pos_t, out_dtype=out_dtype)
    torch.cuda.synchronize()
    got = to_np(out)
    kc_g = kc.cpu().view(torch.int16).numpy().view(np.uint16)
    vc_g = vc.cpu().view(torch.int16).numpy().view(np.uint16)
    for s in range(B):
        pos = int(inp["positions"][s])
        kref = inp["k_cache"][s].copy()
        vref = inp["v_cache"][s].copy()
        O.gqa_append_kv_seq(O.bf16_to_f32(inp["k_new"][s])[None], O.bf16_to_f32(inp["v_new"][s])[None],
                            p["k_norm_w"], kref, vref, O.BF16, start_pos=pos)
        ref = O.gqa_attend(O.bf16_to_f32(inp["q_gate"][s]), p["q_norm_w"], kref, vref, O.BF16, pos)
        if out_dtype == torch.bfloat16:
            assert_bf16_output_close(got[s], ref)
        else:
            assert_f32_output_close(got[s], ref)
        # cache: only row `pos` changed, and to within one bf16 ulp
        mask = np.ones(max_ctx, bool)
        mask[pos] = False
        assert np.array_equal(kc_g[s][mask], inp["k_cache"][s][mask])
        assert np.array_equal(vc_g[s][mask], inp["v_cache"][s][mask])
        assert np.array_equal(vc_g[s][pos], vref[pos])
        kr = O.bf16_to_f32(kref[pos])
        assert np.all(np.abs(O.bf16_to_f32(kc_g[s][pos]) - kr) <= np.maximum(bf16_ulp(kr), 2.0 ** -16))


def test_gqa_decode_batch1_full_context(hip):
    _run_case(hip, [8192], 8192)


def test_gqa_decode_edges(hip):
    # L = 1 (pos 0), chunk boundaries of the split, and odd lengths
    _run_case(hip, [1, 2, 15, 16, 17, 63, 64, 65, 127, 128, 129, 1000, 2047, 2048], 2048)


@pytest.mark.parametrize("B", [8, 32])
def test_gqa_decode_batch_random_lengths(hip, B):
    rng = np.random.default_rng(B)
    _run_case(hip, rng.integers(1, 8193, B), 8192, out_dtype=torch.bfloat16, seed=B)


def test_gqa_decode_long_context(hip):
    # 64K context at two positions (batch 2: 256 chunks per sequence)
    _run_case(hip, [65536, 40000], 65536)


def test_gqa_decode_config4_shape(hip):
    # config 4's batch-16 decode at 32K context: 256-position chunks, 128 per
    # sequence and kv head, the full-dims combine
    rng = np.random.default_rng(16)
    lengths = list(rng.integers(1, 32769, 14)) + [32768, 257]
    _run_case(hip, lengths, 32768, out_dtype=torch.bfloat16, seed=16)


@pytest.mark.parametrize("B", [3, 10, 65, 130])
def test_gqa_decode_position_outside_cache(hip, B):
    """A sequence whose position lies outside the cache (negative or >=
    max_ctx) gets NaN outputs and leaves its cache rows untouched; the other
    sequences of the batch are unaffected (both combine shapes: B <= 8 and
    B > 8). Batches above 64 take the split's multi-pass path (the
    per-64 sums and the prefix carried across blocks of 64 sequences), with
    such zero-work sequences on both sides of the block boundaries."""
    import qff
    max_ctx = 512
    print(f"gqa_decode invalid positions B={B}", flush=True)
    p = synth.gqa_params()
    if B <= 10:
        lengths = [200 + 30 * i for i in range(B)]
    else:
        lengths = list(np.random.default_rng(B).integers(1, max_ctx + 1, B))
    inp = synth.gqa_decode_inputs(B, max_ctx, seed=70 + B, lengths=lengths)
    bad = {1: -1, B - 1: max_ctx}
    if B > 64:
        bad.update({63: -5, 64: max_ctx + 7, 65 % B: 1 << 30, B // 2: -1})
    positions = inp["positions"].copy()
    for s_, v in bad.items():
        positions[s_] = v
    ctx = qff.Context(max_batch=B, max_ctx=max_ctx, max_prefill_tokens=1)
    kc, vc = bf16_tensor(inp["k_cache"]), bf16_tensor(inp["v_cache"])
    out = qff.gqa_decode(ctx, {k: f32_tensor(v) for k, v in p.items()}, bf16_tensor(inp["q_gate"]),
                         bf16_tensor(inp["k_new"]), bf16_tensor(inp["v_new"]), kc, vc,
                         torch.from_numpy(positions).to(DEV), out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = to_np(out)
    kc_g = kc.cpu().view(torch.int16).numpy().view(np.uint16)
    vc_g = vc.cpu().view(torch.int16).numpy().view(np.uint16)
    for s_ in range(B):
        if s_ in bad:
            assert np.isnan(got[s_]).all()
            assert np.array_equal(kc_g[s_], inp["k_cache"][s_]) and np.array_equal(vc_g[s_], inp["v_cache"][s_])
            continue
        pos = int(positions[s_])
        kref, vref = inp["k_cache"][s_].copy(), inp["v_cache"][s_].copy()
        O.gqa_append_kv_seq(O.bf16_to_f32(inp["k_new"][s_])[None], O.bf16_to_f32(inp["v_new"][s_])[None],
                            p["k_norm_w"], kref, vref, O.BF16, start_pos=pos)
        ref = O.gqa_attend(O.bf16_to_f32(inp["q_gate"][s_]), p["q_norm_w"], kref, vref, O.BF16, pos)
        assert_f32_output_close(got[s_], ref)


@pytest.mark.parametrize("L", [65536, 50001])
def test_gqa_decode_batch1_long_context(hip, L):
    # config 4's single-sequence decode: batch 1 spreads the split over 512
    # chunks per kv head
    _run_case(hip, [L], 65536, out_dtype=torch.bfloat16, seed=L)


def test_kv_append_and_gate_kats(hip):
    """The reference's own GPU KATs (QwenFP16AttentionBridgeTests.swift:8-86)
    through qff_kv_append and qff_attention_gate."""
    import ctypes
    import json
    import os
    import qff
    from qff._lib import check, lib
    kats = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))
    k = kats["kv_writer"]
    ctx = qff.Context(max_batch=1, max_ctx=16, max_prefill_tokens=1)
    kin = f32_tensor(np.array(k["k"], np.float32))
    vin = f32_tensor(np.array(k["v"], np.float32))
    for dt, code in ((torch.float16, 2), (torch.bfloat16, 1)):
        kc = torch.zeros(k["max_seq"], 2, 256, dtype=dt, device=DEV)
        vc = torch.zeros_like(kc)
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        check("qff_kv_append", lib().qff_kv_append(ctx.handle, st, ctypes.c_void_p(kin.data_ptr()),
                                                   ctypes.c_void_p(vin.data_ptr()),
                                                   ctypes.c_void_p(kc.data_ptr()),
                                                   ctypes.c_void_p(vc.data_ptr()), code,
                                                   k["position"], k["max_seq"]))
        torch.cuda.synchronize()
        kb = kc.cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1)
        vb = vc.cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1)
        off = k["token_offset"]
        assert np.all(kb[:off] == 0) and np.all(vb[:off] == 0) and np.all(kb[off + 512:] == 0)
        if code == 2:
            assert kb[off:off + 512].tolist() == k["k_f16_bits"]
            assert vb[off:off + 512].tolist() == k["v_f16_bits"]
        else:
            assert np.array_equal(kb[off:off + 512], O.f32_to_bf16(np.array(k["k"], np.float32)))
    g = kats["attention_gate"]
    att = torch.from_numpy(np.array(g["attention_f16_bits"], np.uint16).view(np.int16)).to(DEV)
    gate = f32_tensor(np.array(g["gate"], np.float32))
    out = torch.empty(4, device=DEV)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    check("qff_attention_gate", lib().qff_attention_gate(ctx.handle, st, ctypes.c_void_p(att.data_ptr()),
                                                         ctypes.c_void_p(gate.data_ptr()),
                                                         ctypes.c_void_p(out.data_ptr()), 4))
    torch.cuda.synchronize()
    assert np.all(np.abs(to_np(out) - np.array(g["expected"])) < g["tol"])


def _prefill_case(hip, T, start, max_ctx, rows=None, out_dtype=torch.bfloat16, seed=21):
    import qff
    print(f"gqa_prefill T={T} start={start} max_ctx={max_ctx}", flush=True)
    rng = np.random.default_rng(seed)
    p = synth.gqa_params()
    qg = O.f32_to_bf16(rng.standard_normal((T, 16, 512)).astype(np.float32))
    kk = O.f32_to_bf16(rng.standard_normal((T, 2, 256)).astype(np.float32))
    vv = O.f32_to_bf16(rng.standard_normal((T, 2, 256)).astype(np.float32))
    kc0 = O.f32_to_bf16(rng.standard_normal((max_ctx, 2, 256)).astype(np.float32))
    vc0 = O.f32_to_bf16(rng.standard_normal((max_ctx, 2, 256)).astype(np.float32))
    ctx = qff.Context(max_batch=1, max_ctx=max_ctx, max_prefill_tokens=T)
    kc, vc = bf16_tensor(kc0), bf16_tensor(vc0)
    pg = {k: f32_tensor(v) for k, v in p.items()}
    out = qff.gqa_prefill(ctx, pg, bf16_tensor(qg), bf16_tensor(kk), bf16_tensor(vv), kc, vc,
                          start_pos=start, out_dtype=out_dtype)
    torch.cuda.synchronize()
    got = to_np(out)
    kref, vref = kc0.copy(), vc0.copy()
    O.gqa_append_kv_seq(O.bf16_to_f32(kk), O.bf16_to_f32(vv), p["k_norm_w"], kref, vref, O.BF16,
                        start_pos=start)
    kc_g = kc.cpu().view(torch.int16).numpy().view(np.uint16)
    vc_g = vc.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(vc_g, vref)
    outside = np.ones(max_ctx, bool)
    outside[start:start + T] = False
    assert np.array_equal(kc_g[outside], kc0[outside])
    kr = O.bf16_to_f32(kref[start:start + T])
    assert np.all(np.abs(O.bf16_to_f32(kc_g[start:start + T]) - kr) <= np.maximum(bf16_ulp(kr), 2.0 ** -16))
    for t in (range(T) if rows is None else rows):
        ref = O.gqa_attend(O.bf16_to_f32(qg[t]), p["q_norm_w"], kref, vref, O.BF16, start + t)
        if out_dtype == torch.bfloat16:
            assert_bf16_output_close(got[t], ref)
        else:
            assert_f32_output_close(got[t], ref)


@pytest.mark.parametrize("T,start", [(1, 0), (17, 0), (100, 0), (64, 0), (64, 37), (128, 64), (300, 1000),
                                     (16, 2032)])
def test_gqa_prefill_matches_token_by_token(hip, T, start):
    _prefill_case(hip, T, start, max_ctx=2048, out_dtype=torch.float32 if T == 17 else torch.bfloat16)


def test_gqa_prefill_config3_full_length_sampled_rows(hip):
    """T = 8192 from position 0: every appended K/V entry, and a sample of
    output rows (first, last, tile and block boundaries, random)."""
    rows = sorted({0, 1, 15, 16, 31, 32, 33, 1000, 4095, 4096, 8190, 8191} |
                  set(np.random.default_rng(3).integers(0, 8192, 6).tolist()))
    _prefill_case(hip, 8192, 0, max_ctx=8192, rows=rows)


def test_gqa_rejects_bad_calls(hip):
    """Host-side checks: nothing is launched for the refused calls."""
    import qff
    max_ctx = 64
    ctx = qff.Context(max_batch=2, max_ctx=max_ctx, max_prefill_tokens=8)
    pg = {k: f32_tensor(v) for k, v in synth.gqa_params().items()}
    kc = torch.zeros(max_ctx, 2, 256, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)

    def prefill(T, start):
        qg = torch.zeros(T, 16, 512, dtype=torch.bfloat16, device=DEV)
        kv = torch.zeros(T, 2, 256, dtype=torch.bfloat16, device=DEV)
        return qff.gqa_prefill(ctx, pg, qg, kv, kv, kc, vc, start)

    with pytest.raises(qff.QffError) as e:       # T above max_prefill_tokens
        prefill(16, 0)
    assert e.value.status == -4
    with pytest.raises(qff.QffError) as e:       # past the end of the cache
        prefill(8, 60)
    assert e.value.status == -1
    # a longer cache than the context's max_ctx, written past it: refused for
    # either cache type (the attention's copies of the cache live in the
    # workspace); up to it: accepted
    qg8 = torch.zeros(8, 16, 512, dtype=torch.bfloat16, device=DEV)
    kv8 = torch.zeros(8, 2, 256, dtype=torch.bfloat16, device=DEV)
    for dt in (torch.bfloat16, torch.float16):
        kc_long = torch.zeros(2 * max_ctx, 2, 256, dtype=dt, device=DEV)
        with pytest.raises(qff.QffError) as e:
            qff.gqa_prefill(ctx, pg, qg8, kv8, kv8, kc_long, kc_long.clone(), max_ctx - 4)
        assert e.value.status == -4
        qff.gqa_prefill(ctx, pg, qg8, kv8, kv8, kc_long, kc_long.clone(), max_ctx - 8)
    torch.cuda.synchronize()
    qg = torch.zeros(3, 16, 512, dtype=torch.bfloat16, device=DEV)
    kn = torch.zeros(3, 2, 256, dtype=torch.bfloat16, device=DEV)
    kc3 = torch.zeros(3, max_ctx, 2, 256, dtype=torch.bfloat16, device=DEV)
    pos = torch.zeros(3, dtype=torch.int32, device=DEV)
    with pytest.raises(qff.QffError) as e:       # batch above max_batch
        qff.gqa_decode(ctx, pg, qg, kn, kn, kc3, kc3.clone(), pos)
    assert e.value.status == -4
    # softmax scale and RoPE theta must be finite and positive
    kc2 = torch.zeros(2, max_ctx, 2, 256, dtype=torch.bfloat16, device=DEV)
    for bad in (0.0, -1.0 / 16, float("nan"), float("inf")):
        with pytest.raises(qff.QffError) as e:
            qff.gqa_decode(ctx, pg, qg[:2], kn[:2], kn[:2], kc2, kc2.clone(), pos[:2], scale=bad)
        assert e.value.status == -1
        with pytest.raises(qff.QffError) as e:
            qff.gqa_prefill(ctx, pg, qg[:2], kn[:2], kn[:2], kc, vc, 0, scale=bad)
        assert e.value.status == -1
    with pytest.raises(qff.QffError) as e:
        qff.gqa_decode(ctx, pg, qg[:2], kn[:2], kn[:2], kc2, kc2.clone(), pos[:2], theta=float("inf"))
    assert e.value.status == -1


def test_gqa_decode_f32_inputs(hip):
    """fp32 q_gate / k_new / v_new (in_dtype F32) at random lengths, against
    the oracle fed the same fp32 values."""
    import qff
    B, max_ctx = 5, 4096
    print(f"gqa_decode f32 inputs B={B}", flush=True)
    rng = np.random.default_rng(55)
    p = synth.gqa_params()
    inp = synth.gqa_decode_inputs(B, max_ctx, seed=55, lengths=[1, 700, 4096, 33, 2500])
    qg = rng.standard_normal((B, 16, 512)).astype(np.float32)
    kn = rng.standard_normal((B, 2, 256)).astype(np.float32)
    vn = rng.standard_normal((B, 2, 256)).astype(np.float32)
    ctx = qff.Context(max_batch=B, max_ctx=max_ctx, max_prefill_tokens=1)
    kc, vc = bf16_tensor(inp["k_cache"]), bf16_tensor(inp["v_cache"])
    out = qff.gqa_decode(ctx, {k: f32_tensor(v) for k, v in p.items()}, f32_tensor(qg), f32_tensor(kn),
                         f32_tensor(vn), kc, vc, torch.from_numpy(inp["positions"]).to(DEV),
                         out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = to_np(out)
    kc_g = kc.cpu().view(torch.int16).numpy().view(np.uint16)
    for s in range(B):
        pos = int(inp["positions"][s])
        kref, vref = inp["k_cache"][s].copy(), inp["v_cache"][s].copy()
        O.gqa_append_kv_seq(kn[s][None], vn[s][None], p["k_norm_w"], kref, vref, O.BF16, start_pos=pos)
        ref = O.gqa_attend(qg[s], p["q_norm_w"], kref, vref, O.BF16, pos)
        assert_f32_output_close(got[s], ref)
        kr = O.bf16_to_f32(kref[pos])
        assert np.all(np.abs(O.bf16_to_f32(kc_g[s][pos]) - kr) <= np.maximum(bf16_ulp(kr), 2.0 ** -16))


@pytest.mark.parametrize("T,start", [(100, 37), (300, 0)])
def test_gqa_prefill_f32_inputs(hip, T, start):
    """fp32 q_gate / k / v through the causal prefill, every row against the
    token-by-token oracle fed the same fp32 values."""
    import qff
    print(f"gqa_prefill f32 inputs T={T} start={start}", flush=True)
    max_ctx = 1024
    rng = np.random.default_rng(70 + T)
    p = synth.gqa_params()
    qg = rng.standard_normal((T, 16, 512)).astype(np.float32)
    kk = rng.standard_normal((T, 2, 256)).astype(np.float32)
    vv = rng.standard_normal((T, 2, 256)).astype(np.float32)
    kc0 = O.f32_to_bf16(rng.standard_normal((max_ctx, 2, 256)).astype(np.float32))
    vc0 = O.f32_to_bf16(rng.standard_normal((max_ctx, 2, 256)).astype(np.float32))
    ctx = qff.Context(max_batch=1, max_ctx=max_ctx, max_prefill_tokens=T)
    kc, vc = bf16_tensor(kc0), bf16_tensor(vc0)
    out = qff.gqa_prefill(ctx, {k: f32_tensor(v) for k, v in p.items()}, f32_tensor(qg), f32_tensor(kk),
                          f32_tensor(vv), kc, vc, start_pos=start, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    got = to_np(out)
    kref, vref = kc0.copy(), vc0.copy()
    O.gqa_append_kv_seq(kk, vv, p["k_norm_w"], kref, vref, O.BF16, start_pos=start)
    assert np.array_equal(vc.cpu().view(torch.int16).numpy().view(np.uint16), vref)
    for t in range(T):
        ref = O.gqa_attend(qg[t], p["q_norm_w"], kref, vref, O.BF16, start + t)
        assert_bf16_output_close(got[t], ref)


def _attend_all_rows_torch(qg, kref, vref, q_norm_w, T, theta=1e7, scale=1.0 / 16, eps=1e-6):
    """Every output row of a causal prefill from position 0 in the oracle's
    arithmetic (gqa_attend: per-head RMSNorm of q, RoPE on dims 0..63 with
    host fp32 inverse frequencies, q rounded to fp16, fp32 softmax over
    positions 0..t, output rounded to fp16, times sigmoid(gate)), vectorised
    on the GPU in fp32. qg [T, 16, 512] f32; kref, vref [T, 2, 256] bf16 bits
    (the cache after the append). Pinned against the oracle's gqa_attend on
    sampled rows by the caller."""
    dev = DEV
    q = torch.from_numpy(qg[:, :, :256].copy()).to(dev)
    gate = torch.from_numpy(qg[:, :, 256:].copy()).to(dev)
    w = torch.from_numpy(q_norm_w.astype(np.float32)).to(dev)
    q = q * torch.rsqrt((q * q).mean(-1, keepdim=True) + eps) * w
    inv = torch.from_numpy(np.array([np.float32(1.0) / np.power(np.float32(theta), np.float32(2 * i) / np.float32(64))
                                     for i in range(32)], np.float32)).to(dev)
    ang = torch.arange(T, device=dev, dtype=torch.float32)[:, None] * inv[None, :]
    c, s = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
    x0, x1 = q[:, :, :32].clone(), q[:, :, 32:64].clone()
    q[:, :, :32] = x0 * c - x1 * s
    q[:, :, 32:64] = x1 * c + x0 * s
    q = q.half().float()
    K = torch.from_numpy(O.bf16_to_f32(kref[:T])).to(dev)
    V = torch.from_numpy(O.bf16_to_f32(vref[:T])).to(dev)
    out = torch.empty(T, 16, 256, device=dev)
    mask = torch.triu(torch.ones(T, T, dtype=torch.bool, device=dev), diagonal=1)
    for h in range(16):
        kh = K[:, h // 8, :].contiguous()
        sc = (q[:, h, :].contiguous() @ kh.t().contiguous()) * scale
        sc.masked_fill_(mask, float("-inf"))
        pr = torch.softmax(sc, dim=-1)
        out[:, h, :] = pr @ V[:, h // 8, :].contiguous()
        del sc, pr
    return (out.half().float() * torch.sigmoid(gate)).cpu().numpy()


def test_gqa_prefill_config3_exact_call(hip):
    """Config 3 as bench.py times it: the three-part Q4 GEMM (q|gate 8192,
    k 512, v 512 rows from hidden 2048, fp16 scales) over T = 8192 tokens in
    one call, then qff_gqa_prefill on its bf16 outputs from position 0.
    Projections: 64 sampled tokens of every part against the fp64 product of
    the dequantized weights, each bf16 output within one bf16 ulp plus
    2.5e-3 of its row's RMS (fp16 operands). Attention:
    all 8192 output rows against a vectorised fp32 restatement of the
    oracle's arithmetic, itself checked against the oracle on 8 rows."""
    import qff
    T, H = 8192, 2048
    print("config 3 exact call: Q4 GEMM T=8192 + gqa_prefill", flush=True)
    rng = np.random.default_rng(3)
    xb = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    ws = [synth.q4_weight(rows, H, seed=300 + i) for i, rows in enumerate((8192, 512, 512))]
    parts = [(torch.from_numpy(w.view(np.int32)).to(DEV), torch.from_numpy(s.view(np.int16)).view(torch.float16).to(DEV),
              torch.from_numpy(b.view(np.int16)).view(torch.float16).to(DEV)) for w, s, b in ws]
    ctx = qff.Context(max_batch=1, max_ctx=T, max_prefill_tokens=T)
    qg = torch.empty(T, 8192, dtype=torch.bfloat16, device=DEV)
    k = torch.empty(T, 512, dtype=torch.bfloat16, device=DEV)
    v = torch.empty(T, 512, dtype=torch.bfloat16, device=DEV)
    qff.q4_matmul_parts(ctx, parts, bf16_tensor(xb), outs=(qg, k, v))
    p = synth.gqa_params()
    kc = torch.zeros(T, 2, 256, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    out = qff.gqa_prefill(ctx, {kk: f32_tensor(vv) for kk, vv in p.items()}, qg.view(T, 16, 512),
                          k.view(T, 2, 256), v.view(T, 2, 256), kc, vc, 0, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    # projections on sampled tokens: the GEMM's fp16 operands (W rounded once
    # to 11 significant bits) put ~3e-4 of each row's RMS of noise on every
    # output (absolute, so it dominates near zero), then rounded once to bf16
    toks = sorted({0, 1, 127, 128, 4095, 4096, 8191} | set(rng.integers(0, T, 57).tolist()))
    xs = O.bf16_to_f32(xb[toks]).astype(np.float64)
    for (w, s, b), y in zip(ws, (qg, k, v)):
        ref = xs @ O.q4_dequant(w, s, b, O.F16).astype(np.float64).T
        got = to_np(y)[toks]
        rms = np.sqrt((ref * ref).mean(axis=1, keepdims=True))
        err = (np.abs(got - ref) - bf16_ulp(ref)) / rms
        assert np.all(err <= 2.5e-3), f"Q4 GEMM output beyond one bf16 ulp + 2.5e-3 RMS: worst {err.max():.3g}"
    print("  projections ok", flush=True)
    qg_f = to_np(qg).reshape(T, 16, 512)
    kref = np.zeros((T, 2, 256), np.uint16)
    vref = np.zeros((T, 2, 256), np.uint16)
    O.gqa_append_kv_seq(to_np(k).reshape(T, 2, 256), to_np(v).reshape(T, 2, 256), p["k_norm_w"], kref, vref,
                        O.BF16, start_pos=0)
    assert np.array_equal(vc.cpu().view(torch.int16).numpy().view(np.uint16), vref)
    kr = O.bf16_to_f32(kref)
    assert np.all(np.abs(O.bf16_to_f32(kc.cpu().view(torch.int16).numpy().view(np.uint16)) - kr)
                  <= np.maximum(bf16_ulp(kr), 2.0 ** -16))
    ref_all = _attend_all_rows_torch(qg_f, kref, vref, p["q_norm_w"], T)
    for t in (0, 1, 63, 64, 4095, 5000, 8190, 8191):
        o = O.gqa_attend(qg_f[t], p["q_norm_w"], kref, vref, O.BF16, t)
        # both round the attention output to fp16 from fp32 sums taken in a
        # different order: at most a couple of fp16 ulps (2^-10 |x|) apart
        assert np.all(np.abs(o - ref_all[t]) <= np.maximum(2e-3, np.abs(o) * 2.0 ** -9)), \
            f"vectorised restatement off the oracle at row {t}"
    print("  restatement pinned; checking all rows", flush=True)
    assert_bf16_output_close(to_np(out), ref_all)


def test_gqa_prefill_config3_from_x_end_to_end(hip):
    """Config 3 from its input X, each side on its own projections: the HIP
    path (the three-part Q4 GEMM on fp16 operands, bf16 outputs, then
    qff_gqa_prefill from position 0) against the oracle's own chain
    (QwenQ4ActiveExpertStreamingRunner.swift:1041-1150): the reference's
    fp32 factored Q4 product (deltanet.metal:1838-1895) of X for q|gate at
    the sampled rows and for k, v at every position (the fp64 product of the
    dequantized weights, pinned to the factored order on the sampled rows),
    rounded to bf16 as the workload's Q/K/V are, then the oracle's
    append and attention. First the projections: every k / v / q|gate value
    the GEMM produced is within one bf16 ulp plus 2.5e-3 of its row's RMS of
    the oracle's (the fp16-weight error). Then the attention outputs of the
    sampled rows, in two links: against the oracle's attention fed the
    GPU's own bf16 projections, the plain bar (max-abs 2e-2, or one bf16 ulp
    of the output); against the oracle's own chain, that bar plus two bf16
    ulps of the largest |V| the output mixes (per head and dim over the
    attended positions): the GEMM's error (~3e-4 of a row's RMS, under the
    2^-9 of the bf16 the workload stores Q/K/V in) makes a few percent of the
    two sides' projections round to neighbouring bf16 values, and an output
    that few positions dominate moves with their V by up to an ulp of V, not
    of itself. The median end-to-end error is under one bf16 ulp of the
    output."""
    import qff
    T, H = 8192, 2048
    print("config 3 from X: Q4 GEMM T=8192 + gqa_prefill vs the oracle's own projections", flush=True)
    rng = np.random.default_rng(33)
    xb = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    ws = [synth.q4_weight(rows, H, seed=330 + i) for i, rows in enumerate((8192, 512, 512))]
    parts = [(torch.from_numpy(w.view(np.int32)).to(DEV), torch.from_numpy(s.view(np.int16)).view(torch.float16).to(DEV),
              torch.from_numpy(b.view(np.int16)).view(torch.float16).to(DEV)) for w, s, b in ws]
    ctx = qff.Context(max_batch=1, max_ctx=T, max_prefill_tokens=T)
    qg = torch.empty(T, 8192, dtype=torch.bfloat16, device=DEV)
    k = torch.empty(T, 512, dtype=torch.bfloat16, device=DEV)
    v = torch.empty(T, 512, dtype=torch.bfloat16, device=DEV)
    qff.q4_matmul_parts(ctx, parts, bf16_tensor(xb), outs=(qg, k, v))
    p = synth.gqa_params()
    kc = torch.zeros(T, 2, 256, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    out = qff.gqa_prefill(ctx, {kk: f32_tensor(vv) for kk, vv in p.items()}, qg.view(T, 16, 512),
                          k.view(T, 2, 256), v.view(T, 2, 256), kc, vc, 0, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    got = to_np(out)
    x = O.bf16_to_f32(xb)
    rows = [0, 1, 63, 64, 511, 4095, 4096, 6000, 8190, 8191]
    # the oracle's projections: k, v of every position (fp64 dense product),
    # the reference's fp32 factored order at the sampled rows
    dense = [O.q4_dequant(w, s, b, O.F16).astype(np.float64) for w, s, b in ws]
    k_ref = (x.astype(np.float64) @ dense[1].T).astype(np.float32)
    v_ref = (x.astype(np.float64) @ dense[2].T).astype(np.float32)
    for t in rows:
        for part, full in ((1, k_ref), (2, v_ref)):
            fac = O.q4_matvec(*ws[part], x[t])
            assert np.max(np.abs(fac - full[t])) <= 1e-5 * np.max(np.abs(full[t])), "factored order vs fp64"
    print("  oracle projections ready", flush=True)
    for gpu, ref in ((k, k_ref), (v, v_ref)):
        g_ = to_np(gpu)
        rms = np.sqrt((ref.astype(np.float64) ** 2).mean(axis=1, keepdims=True))
        err = (np.abs(g_ - ref) - bf16_ulp(ref)) / rms
        assert np.all(err <= 2.5e-3), f"k/v projection beyond one bf16 ulp + 2.5e-3 RMS: worst {err.max():.3g}"
    kref = np.zeros((T, 2, 256), np.uint16)
    vref = np.zeros((T, 2, 256), np.uint16)
    O.gqa_append_kv_seq(O.round_bf16(k_ref).reshape(T, 2, 256), O.round_bf16(v_ref).reshape(T, 2, 256),
                        p["k_norm_w"], kref, vref, O.BF16, start_pos=0)
    qg_g = to_np(qg)
    kg_bits = kc.cpu().view(torch.int16).numpy().view(np.uint16)
    vg_bits = vc.cpu().view(torch.int16).numpy().view(np.uint16)
    errs = []
    for t in rows:
        qg_ref = O.q4_matvec(*ws[0], x[t])
        rms = np.sqrt(np.mean(qg_ref.astype(np.float64) ** 2))
        assert np.all(np.abs(qg_g[t] - qg_ref) - bf16_ulp(qg_ref) <= 2.5e-3 * rms), f"q|gate projection row {t}"
        # link 1: the attention on the GPU's own projections
        own = O.gqa_attend(qg_g[t].reshape(16, 512), p["q_norm_w"], kg_bits, vg_bits, O.BF16, t)
        assert_bf16_output_close(got[t], own)
        # link 2: end to end against the oracle's own projections
        ref = O.gqa_attend(O.round_bf16(qg_ref).reshape(16, 512), p["q_norm_w"], kref, vref, O.BF16, t)
        err = np.abs(got[t].astype(np.float64) - ref)
        errs.append(err / bf16_ulp(ref))
        vmax = np.abs(O.bf16_to_f32(vref[:t + 1])).max(axis=0)          # [2, 256]
        vmax = np.repeat(vmax, 8, axis=0)                                 # per q head
        lim = np.maximum(2e-2, bf16_ulp(ref)) + 2 * bf16_ulp(vmax)
        assert np.all(err <= lim), f"row {t}: {int((err > lim).sum())} outside; worst {err.max():.4g}"
    errs = np.concatenate([e.reshape(-1) for e in errs])
    print(f"  {len(rows)} rows within the bar: median error {np.median(errs):.3g} output ulps, "
          f"max {errs.max():.3g}", flush=True)
    assert np.median(errs) <= 1.0
    ctx.close()


def test_gqa_prefill_graph_replay(hip):
    """qff_gqa_prefill captured in a HIP graph (T = 100 at start 37 on a bf16
    cache, so the prep launch writes the fp16 K copy of the 37 older rows and
    the transposed V copy beside the per-token prep) and replayed three
    times, with an eager prefill of another shape on the same context (which
    rewrites the workspace copies) between replays: every replay's output
    and caches equal an eager call's on the same inputs, bit for bit."""
    import qff
    rng = np.random.default_rng(77)
    p = synth.gqa_params()
    pg = {k: f32_tensor(v) for k, v in p.items()}
    T, start, max_ctx = 100, 37, 1024
    qg = bf16_tensor(O.f32_to_bf16(rng.standard_normal((T, 16, 512)).astype(np.float32)))
    kk = bf16_tensor(O.f32_to_bf16(rng.standard_normal((T, 2, 256)).astype(np.float32)))
    vv = bf16_tensor(O.f32_to_bf16(rng.standard_normal((T, 2, 256)).astype(np.float32)))
    kc0 = bf16_tensor(O.f32_to_bf16(rng.standard_normal((max_ctx, 2, 256)).astype(np.float32)))
    vc0 = bf16_tensor(O.f32_to_bf16(rng.standard_normal((max_ctx, 2, 256)).astype(np.float32)))
    ctx = qff.Context(max_batch=1, max_ctx=max_ctx, max_prefill_tokens=256)
    # the eager reference
    kc_ref, vc_ref = kc0.clone(), vc0.clone()
    ref = qff.gqa_prefill(ctx, pg, qg, kk, vv, kc_ref, vc_ref, start_pos=start)
    torch.cuda.synchronize()
    ref = ref.clone()
    # another shape on the same context, run eagerly between replays
    T2 = 70
    o_args = [bf16_tensor(O.f32_to_bf16(rng.standard_normal(s).astype(np.float32)))
              for s in ((T2, 16, 512), (T2, 2, 256), (T2, 2, 256))]
    kc2, vc2 = kc0.clone(), vc0.clone()
    kc, vc = kc0.clone(), vc0.clone()
    out = torch.empty(T, 16, 256, dtype=torch.bfloat16, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        qff.gqa_prefill(ctx, pg, qg, kk, vv, kc.clone(), vc.clone(), start_pos=start, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    print(f"gqa_prefill graph capture T={T} start={start}", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        qff.gqa_prefill(ctx, pg, qg, kk, vv, kc, vc, start_pos=start, out=out)
    for rep in range(3):
        print(f"gqa_prefill graph replay {rep}", flush=True)
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}: output"
        assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref), f"replay {rep}: caches"
        qff.gqa_prefill(ctx, pg, *o_args, kc2, vc2, start_pos=500)
        torch.cuda.synchronize()
