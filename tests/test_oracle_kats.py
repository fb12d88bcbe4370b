"""Pins the oracle to the reference's own known-answer tests (transcribed in
tests/golden/reference_kats.json) and the storage conversions to IEEE RNE."""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def test_matvec_row_major_kat():
    # QwenDeltaNetMathTests.swift:5-12
    k = KATS["matvec"]
    y = O.matvec(np.array(k["weight"], np.float32), np.array(k["vec"], np.float32))
    assert y.tolist() == k["expected"]


def test_rmsnorm_one_plus_w_kat():
    # QwenDeltaNetMathTests.swift:14-21 (the CPU norm multiplies by 1 + w)
    k = KATS["rmsnorm_one_plus_w"]
    y = O.rmsnorm(np.array(k["input"], np.float32), np.array(k["weight"], np.float32),
                  eps=k["eps"], one_plus_w=True)
    assert np.all(np.abs(y - np.array(k["expected"])) < k["tol"])
    # the Metal convention (w, not 1 + w) gives a different answer: the KAT
    # distinguishes the two, so a swapped flag fails here
    y2 = O.rmsnorm(np.array(k["input"], np.float32), np.array(k["weight"], np.float32),
                   eps=k["eps"], one_plus_w=False)
    assert np.max(np.abs(y2 - np.array(k["expected"]))) > 0.1


def test_rmsnorm_zero_kat():
    # QwenDeltaNetMathTests.swift:23-28
    k = KATS["rmsnorm_zero"]
    y = O.rmsnorm(np.array(k["input"], np.float32), np.array(k["weight"], np.float32),
                  eps=k["eps"], one_plus_w=True)
    assert y.tolist() == k["expected"]


@pytest.mark.parametrize("dtype", [O.F16, O.BF16])
def test_kv_writer_token_major_kat(dtype):
    # QwenFP16AttentionBridgeTests.swift:8-52 (F16 as the reference; BF16 is
    # the same layout with the build's cache dtype)
    k = KATS["kv_writer"]
    S, H, D = k["max_seq"], k["num_kv_heads"], k["head_dim"]
    kc = np.zeros((S, H, D), np.uint16)
    vc = np.zeros((S, H, D), np.uint16)
    kin = np.array(k["k"], np.float32)
    vin = np.array(k["v"], np.float32)
    O.kv_append(kin, vin, kc, vc, dtype, k["position"])
    off = k["token_offset"]
    kf, vf = kc.reshape(-1), vc.reshape(-1)
    assert np.all(kf[:off] == 0) and np.all(vf[:off] == 0)
    if dtype == O.F16:
        assert kf[off:off + 512].tolist() == k["k_f16_bits"]
        assert vf[off:off + 512].tolist() == k["v_f16_bits"]
    else:
        assert np.array_equal(kf[off:off + 512], O.f32_to_bf16(kin))
        assert np.array_equal(vf[off:off + 512], O.f32_to_bf16(vin))
    assert np.all(kf[off + 512:] == 0)


def test_attention_gate_kat():
    # QwenFP16AttentionBridgeTests.swift:54-86
    k = KATS["attention_gate"]
    y = O.attention_gate(np.array(k["attention_f16_bits"], np.uint16),
                         np.array(k["gate"], np.float32))
    assert np.all(np.abs(y - np.array(k["expected"])) < k["tol"])


def test_f16_conversion_matches_ieee_rne(rng):
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(100),
        rng.standard_normal(5000).astype(np.float32) * np.float32(1e-5),  # subnormals
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e9, -1e9, 6.1e-5, 5.96e-8, 2.98e-8,
                  1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32),
    ])
    L = O.lib()
    ours = np.array([L.qffo_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(ours, x.astype(np.float16).view(np.uint16))
    back = np.array([L.qffo_f16_to_f32(int(b)) for b in ours], np.float32)
    assert np.array_equal(back, x.astype(np.float16).astype(np.float32))


def test_bf16_conversion_rne():
    L = O.lib()
    # 1 + 2^-8 is exactly halfway between bf16 1.0 and 1.0078125: ties to even
    cases = {1.0: 0x3F80, 1.0 + 2.0 ** -8: 0x3F80, 1.0 + 3 * 2.0 ** -8: 0x3F82,
             -2.0: 0xC000, 1.0 + 2.0 ** -8 + 2.0 ** -20: 0x3F81}
    for v, bits in cases.items():
        assert L.qffo_f32_to_bf16(v) == bits
        assert O.f32_to_bf16(np.array([v], np.float32))[0] == bits
    x = np.random.default_rng(1).standard_normal(10000).astype(np.float32)
    ours = np.array([L.qffo_f32_to_bf16(float(v)) for v in x], np.uint16)
    assert np.array_equal(ours, O.f32_to_bf16(x))
    # bf16 -> f32 is exact: the round trip of representable values is identity
    assert np.array_equal(O.round_bf16(O.bf16_to_f32(ours)), O.bf16_to_f32(ours))


def test_dense_arena_layout_kat():
    # QwenGenerationSupportTests.swift:7-9: the arena ends 32 KiB after the
    # last bias block; the attention rows' Q4 blocks (qkv/z/b/a/out, k, v)
    # are each w (rows*cols/2 B) then scales, biases (rows*cols/64*2 B).
    a = KATS["dense_arena"]
    assert a["totalByteLength"] == a["shDownBOff"] + 32_768

    def block(rows, cols):
        return rows * cols // 2, rows * cols // 64 * 2

    w, sb = block(8192, 2048)
    assert a["qkvSOff"] - a["qkvWOff"] == w and a["qkvBOff"] - a["qkvSOff"] == sb
    w, sb = block(4096, 2048)
    assert a["zSOff"] - a["zWOff"] == w and a["zBOff"] - a["zSOff"] == sb
    w, sb = block(2048, 4096)
    assert a["linOutSOff"] - a["linOutWOff"] == w and a["linOutBOff"] - a["linOutSOff"] == sb
    w, sb = block(512, 2048)
    assert a["kProjSOff"] - a["kProjWOff"] == w and a["vProjSOff"] - a["vProjWOff"] == w
