"""Writes tests/golden/reference_kats.json: the known-answer vectors that the
reference's own test suite holds for this path, transcribed as data.

Sources (reference paths under Tests/QwenFieldfareCore/):
  QwenDeltaNetMathTests.swift:5-12   matVecMul row-major -> [9, 21]
  QwenDeltaNetMathTests.swift:14-21  rmsNorm (1 + w), eps 0 -> [1.6970563, 3.3941126]
  QwenDeltaNetMathTests.swift:23-28  rmsNorm of zeros -> zeros
  Kernels/Attention/QwenFP16AttentionBridgeTests.swift:8-52
        KV writer: k_i = i/64 - 4, v_i = 3 - i/80 (i < 512), position 1,
        max sequence 3, token-major [seq, 2, 256] FP16 cache: entries before
        offset 512 stay zero, entries 512.. hold Float16(k_i), Float16(v_i)
  Kernels/Attention/QwenFP16AttentionBridgeTests.swift:54-86
        gate: attention FP16 [0.5, -1, 2, -3], gate [-2, -0.5, 0.5, 2]
        -> attention / (1 + exp(-gate)), tolerance 1e-5
  QwenGenerationSupportTests.swift:7-9
        DenseLayerArena.totalByteLength == shDownBOff + 32_768, with the
        arena offsets of Runtime/Generation/QwenQ4ActiveExpertStreamingRunner.swift:15-51

Expected FP16 bit patterns are IEEE binary16 round-to-nearest-even of the
listed float32 inputs (numpy's float16 cast), as Swift's Float16(x) is.
Run: python tests/golden/make_reference_kats.py
"""
import json
import os

import numpy as np

k = np.array([np.float32(i) / np.float32(64.0) - np.float32(4.0) for i in range(512)], np.float32)
v = np.array([np.float32(3.0) - np.float32(i) / np.float32(80.0) for i in range(512)], np.float32)
attn = np.array([0.5, -1.0, 2.0, -3.0], np.float16)
gate = np.array([-2.0, -0.5, 0.5, 2.0], np.float32)
gate_expected = attn.astype(np.float64) / (1.0 + np.exp(-gate.astype(np.float64)))

arena = {  # QwenQ4ActiveExpertStreamingRunner.swift:9-51
    "totalByteLength": 22_456_448,
    "qkvWOff": 0, "qkvSOff": 8_388_608, "qkvBOff": 8_912_896,
    "zWOff": 9_437_184, "zSOff": 13_631_488, "zBOff": 13_893_632,
    "bWOff": 14_155_776, "bSOff": 14_188_544, "bBOff": 14_190_592,
    "aWOff": 14_192_640, "aSOff": 14_225_408, "aBOff": 14_227_456,
    "linOutWOff": 14_229_504, "linOutSOff": 18_423_808, "linOutBOff": 18_685_952,
    "kProjWOff": 18_948_096, "kProjSOff": 19_472_384, "kProjBOff": 19_505_152,
    "vProjWOff": 19_537_920, "vProjSOff": 20_062_208, "vProjBOff": 20_094_976,
    "shDownBOff": 22_423_680,
}

kats = {
    "matvec": {"weight": [[1, 2, 3], [4, 5, 6]], "vec": [2, -1, 3], "expected": [9, 21]},
    "rmsnorm_one_plus_w": {"input": [3, 4], "weight": [1, 2], "eps": 0.0,
                           "expected": [1.6970563, 3.3941126], "tol": 1e-5},
    "rmsnorm_zero": {"input": [0, 0, 0], "weight": [1, 1, 1], "eps": 1e-6,
                     "expected": [0, 0, 0]},
    "kv_writer": {"position": 1, "max_seq": 3, "num_kv_heads": 2, "head_dim": 256,
                  "k": k.tolist(), "v": v.tolist(), "token_offset": 512,
                  "k_f16_bits": k.astype(np.float16).view(np.uint16).tolist(),
                  "v_f16_bits": v.astype(np.float16).view(np.uint16).tolist()},
    "attention_gate": {"attention_f16_bits": attn.view(np.uint16).tolist(),
                       "gate": gate.tolist(), "expected": gate_expected.tolist(),
                       "tol": 1e-5},
    "dense_arena": arena,
}

out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kats.json")
with open(out, "w") as f:
    json.dump(kats, f, indent=1)
print("wrote", out)
