"""GPU parity of the fused full-attention entry points on an fp16 KV cache,
the cache type the reference allocates (QwenQ4ActiveExpertStreamingRunner
.swift:731-732) and writes with qwen_update_kv_cache_f16 (deltanet.metal
:670-689): qff_gqa_decode and qff_gqa_prefill with qff_gqa_params.kv_f16 = 1
against the oracle's fp16-cache append and attention (reference order,
half-rounded q and attention output).

Tolerance as for the bf16 cache: outputs max-abs <= 2e-2 (bf16 outputs may
also be one bf16 ulp off where that exceeds 2e-2). The appended v entries
are the fp16 rounding of the same fp32 values on both sides (bit-exact); the
appended k entries are normed and rotated in a different order, so they
agree to one fp16 ulp, or to 2^-18 where the rotation nearly cancels (the
two sides' fp32 cos / sin of angles up to ~6.5e4 rad differ by ~1e-7, more
than an fp16 ulp of a result near zero); every other cache entry is
untouched."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import (DEV, assert_bf16_output_close, assert_f32_output_close, bf16_tensor, f16_tensor,
                      f32_tensor, to_np)
from oracle import oracle as O
from qff import synth

pytestmark = pytest.mark.gpu


def f16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of fp16 values at |x| (2^-24 in the subnormal range)."""
    a = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def k_bar(kr: np.ndarray) -> np.ndarray:
    return np.maximum(f16_ulp(kr), 2.0 ** -18)


def _f16_bits_of_bf16(bits: np.ndarray) -> np.ndarray:
    """A bf16 cache's values as fp16 bits (exact inside fp16's range)."""
    return O.f32_to_f16(O.bf16_to_f32(bits))


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def _decode_case(lengths, max_ctx, out_dtype=torch.float32, seed=11):
    import qff
    B = len(lengths)
    print(f"gqa_decode fp16 cache B={B} max_ctx={max_ctx} lengths={list(lengths)[:8]}", flush=True)
    p = synth.gqa_params()
    inp = synth.gqa_decode_inputs(B, max_ctx, seed=seed, lengths=lengths)
    kc0, vc0 = _f16_bits_of_bf16(inp["k_cache"]), _f16_bits_of_bf16(inp["v_cache"])
    ctx = qff.Context(max_batch=max(B, 1), max_ctx=max_ctx, max_prefill_tokens=1)
    kc, vc = f16_tensor(kc0), f16_tensor(vc0)
    pg = {k: f32_tensor(v) for k, v in p.items()}
    pos_t = torch.from_numpy(inp["positions"]).to(DEV)
    out = qff.gqa_decode(ctx, pg, bf16_tensor(inp["q_gate"]), bf16_tensor(inp["k_new"]),
                         bf16_tensor(inp["v_new"]), kc, vc, pos_t, out_dtype=out_dtype)
    torch.cuda.synchronize()
    got = to_np(out)
    kc_g, vc_g = _u16(kc), _u16(vc)
    for s in range(B):
        pos = int(inp["positions"][s])
        kref, vref = kc0[s].copy(), vc0[s].copy()
        O.gqa_append_kv_seq(O.bf16_to_f32(inp["k_new"][s])[None], O.bf16_to_f32(inp["v_new"][s])[None],
                            p["k_norm_w"], kref, vref, O.F16, start_pos=pos)
        ref = O.gqa_attend(O.bf16_to_f32(inp["q_gate"][s]), p["q_norm_w"], kref, vref, O.F16, pos)
        if out_dtype == torch.bfloat16:
            assert_bf16_output_close(got[s], ref)
        else:
            assert_f32_output_close(got[s], ref)
        mask = np.ones(max_ctx, bool)
        mask[pos] = False
        assert np.array_equal(kc_g[s][mask], kc0[s][mask])
        assert np.array_equal(vc_g[s][mask], vc0[s][mask])
        assert np.array_equal(vc_g[s][pos], vref[pos])
        kr = O.f16_to_f32(kref[pos])
        assert np.all(np.abs(O.f16_to_f32(kc_g[s][pos]) - kr) <= k_bar(kr))


def test_gqa_decode_f16_cache_batch1_full_context(hip):
    _decode_case([8192], 8192)


def test_gqa_decode_f16_cache_edges(hip):
    _decode_case([1, 2, 15, 16, 17, 63, 64, 65, 127, 128, 129, 1000, 2047, 2048], 2048)


@pytest.mark.parametrize("B", [8, 32])
def test_gqa_decode_f16_cache_batch_random_lengths(hip, B):
    rng = np.random.default_rng(100 + B)
    _decode_case(rng.integers(1, 8193, B), 8192, out_dtype=torch.bfloat16, seed=100 + B)


def test_gqa_decode_f16_cache_long_context(hip):
    _decode_case([65536, 40000], 65536)


@pytest.mark.parametrize("T,start,out_dtype", [(1, 0, torch.bfloat16), (100, 0, torch.float32),
                                               (64, 37, torch.bfloat16), (128, 64, torch.bfloat16),
                                               (300, 1000, torch.bfloat16), (16, 2032, torch.bfloat16)])
def test_gqa_prefill_f16_cache_matches_token_by_token(hip, T, start, out_dtype):
    import qff
    max_ctx = 2048
    print(f"gqa_prefill fp16 cache T={T} start={start}", flush=True)
    rng = np.random.default_rng(200 + T)
    p = synth.gqa_params()
    qg = O.f32_to_bf16(rng.standard_normal((T, 16, 512)).astype(np.float32))
    kk = O.f32_to_bf16(rng.standard_normal((T, 2, 256)).astype(np.float32))
    vv = O.f32_to_bf16(rng.standard_normal((T, 2, 256)).astype(np.float32))
    kc0 = O.f32_to_f16(rng.standard_normal((max_ctx, 2, 256)).astype(np.float32))
    vc0 = O.f32_to_f16(rng.standard_normal((max_ctx, 2, 256)).astype(np.float32))
    ctx = qff.Context(max_batch=1, max_ctx=max_ctx, max_prefill_tokens=T)
    kc, vc = f16_tensor(kc0), f16_tensor(vc0)
    pg = {k: f32_tensor(v) for k, v in p.items()}
    out = qff.gqa_prefill(ctx, pg, bf16_tensor(qg), bf16_tensor(kk), bf16_tensor(vv), kc, vc,
                          start_pos=start, out_dtype=out_dtype)
    torch.cuda.synchronize()
    got = to_np(out)
    kref, vref = kc0.copy(), vc0.copy()
    O.gqa_append_kv_seq(O.bf16_to_f32(kk), O.bf16_to_f32(vv), p["k_norm_w"], kref, vref, O.F16,
                        start_pos=start)
    kc_g, vc_g = _u16(kc), _u16(vc)
    assert np.array_equal(vc_g, vref)
    outside = np.ones(max_ctx, bool)
    outside[start:start + T] = False
    assert np.array_equal(kc_g[outside], kc0[outside])
    kr = O.f16_to_f32(kref[start:start + T])
    assert np.all(np.abs(O.f16_to_f32(kc_g[start:start + T]) - kr) <= k_bar(kr))
    for t in range(T):
        ref = O.gqa_attend(O.bf16_to_f32(qg[t]), p["q_norm_w"], kref, vref, O.F16, start + t)
        if out_dtype == torch.bfloat16:
            assert_bf16_output_close(got[t], ref)
        else:
            assert_f32_output_close(got[t], ref)


def test_gqa_rejects_bad_cache_flag(hip):
    """kv_f16 other than 0 or 1, and caches of mixed or other types, are
    refused before anything is launched."""
    import qff
    from qff._lib import GqaParams, lib
    max_ctx = 64
    ctx = qff.Context(max_batch=1, max_ctx=max_ctx, max_prefill_tokens=8)
    pg = {k: f32_tensor(v) for k, v in synth.gqa_params().items()}
    qg = torch.zeros(1, 16, 512, dtype=torch.bfloat16, device=DEV)
    kn = torch.zeros(1, 2, 256, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(1, max_ctx, 2, 256, dtype=torch.float16, device=DEV)
    vc = torch.zeros_like(kc)
    pos = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.zeros(1, 16, 256, dtype=torch.float32, device=DEV)
    prm = GqaParams(pg["q_norm_w"].data_ptr(), pg["k_norm_w"].data_ptr(), 1e7, 64, 1.0 / 16, 1e-6, 2)
    st = lib().qff_gqa_decode(ctx.handle, None, ctypes.byref(prm), qg.data_ptr(), kn.data_ptr(), kn.data_ptr(),
                              qff.BF16, kc.data_ptr(), vc.data_ptr(), pos.data_ptr(), out.data_ptr(), qff.F32,
                              1, max_ctx)
    assert st == -1
    with pytest.raises(TypeError):
        qff.gqa_decode(ctx, pg, qg, kn, kn, kc, vc.to(torch.bfloat16), pos)
    with pytest.raises(TypeError):
        qff.gqa_decode(ctx, pg, qg, kn, kn, kc.float(), vc.float(), pos)
