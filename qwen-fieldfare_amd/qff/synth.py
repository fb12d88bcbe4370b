"""Seeded synthetic inputs at the benchmark configurations.

Distributions follow the workload definitions: activations ~N(0,1) stored as
bf16, fp32 recurrent state ~N(0, 0.02), beta = sigmoid(b) with b ~N(0,1),
g = -exp(A_log) * softplus(a + dt_bias) with A_log ~U(-1,1), dt_bias
~N(0,0.1), conv weights ~N(0,0.5) and norm weights ~1 + N(0,0.1) (both
bf16-representable, as checkpoint tensors are), affine-Q4 weights with
uniform random nibbles, fp16 scales ~U(0.005,0.02) and fp16 biases
~N(0,0.05). Normal "N(m, s)" means standard deviation s.

Arrays are numpy; bf16 tensors are returned as uint16 bit patterns and f16
as uint16 bit patterns too, so the same bytes feed the HIP path and the
oracle.
"""
from __future__ import annotations

import numpy as np

BASE_SEED = 0x5157454E


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _bf16_vals(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _normal(rng, shape, std=1.0, mean=0.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std) + np.float32(mean))


def deltanet_params(seed: int = BASE_SEED):
    """Per-layer constants: A_log, dt_bias [32], conv_w [8192,4], norm_w [128]
    (float32 holding bf16-representable values for conv_w / norm_w)."""
    rng = np.random.default_rng(seed ^ 0xD17A)
    return {
        "a_log": rng.uniform(-1.0, 1.0, 32).astype(np.float32),
        "dt_bias": _normal(rng, 32, 0.1),
        "conv_w": _bf16_vals(_bf16_bits(_normal(rng, (8192, 4), 0.5))),
        "norm_w": _bf16_vals(_bf16_bits(_normal(rng, 128, 0.1, 1.0))),
    }


def deltanet_decode_inputs(batch: int = 1, seed: int = BASE_SEED):
    """Config 0 (batch 1) and the DeltaNet half of config 4: one decode step.
    qkv [B,8192] and z [B,4096] as bf16 bits; a, b [B,32] f32; conv_state
    [B,8192,4] f32 with the 3-token history in slots 1..3 (slot 0 is never
    read); ssm_state [B,32,128,128] f32 (row = v index, column = k index)."""
    rng = np.random.default_rng(seed)
    conv = np.zeros((batch, 8192, 4), np.float32)
    conv[:, :, 1:] = _normal(rng, (batch, 8192, 3))
    return {
        "qkv": _bf16_bits(_normal(rng, (batch, 8192))),
        "z": _bf16_bits(_normal(rng, (batch, 4096))),
        "a": _normal(rng, (batch, 32)),
        "b": _normal(rng, (batch, 32)),
        "conv_state": conv,
        "ssm_state": _normal(rng, (batch, 32, 128, 128), 0.02),
    }


def deltanet_prefill_inputs(T: int = 4096, seed: int = BASE_SEED + 1):
    """Config 1: one sequence of T tokens, zero initial conv and ssm state."""
    rng = np.random.default_rng(seed)
    return {
        "qkv": _bf16_bits(_normal(rng, (T, 8192))),
        "z": _bf16_bits(_normal(rng, (T, 4096))),
        "a": _normal(rng, (T, 32)),
        "b": _normal(rng, (T, 32)),
        "conv_state": np.zeros((8192, 4), np.float32),
        "ssm_state": np.zeros((32, 128, 128), np.float32),
    }


def gqa_params(seed: int = BASE_SEED):
    rng = np.random.default_rng(seed ^ 0x6A0A)
    return {
        "q_norm_w": _bf16_vals(_bf16_bits(_normal(rng, 256, 0.1, 1.0))),
        "k_norm_w": _bf16_vals(_bf16_bits(_normal(rng, 256, 0.1, 1.0))),
    }


def gqa_decode_inputs(batch: int, max_ctx: int = 8192, seed: int = BASE_SEED + 2,
                      lengths=None):
    """Config 2: per-sequence attended length L_b ~U[1, max_ctx] (the new
    token sits at position L_b - 1); bf16 K/V caches [B,max_ctx,2,256]
    ~N(0,1) (entries at and beyond the new position are overwritten or
    unused); q_gate [B,16,512] (per-head interleaved q | gate), k_new,
    v_new [B,2,256] as bf16 bits."""
    rng = np.random.default_rng(seed)
    if lengths is None:
        lengths = rng.integers(1, max_ctx + 1, batch)
    lengths = np.asarray(lengths, np.int32)
    return {
        "positions": (lengths - 1).astype(np.int32),
        "q_gate": _bf16_bits(_normal(rng, (batch, 16, 512))),
        "k_new": _bf16_bits(_normal(rng, (batch, 2, 256))),
        "v_new": _bf16_bits(_normal(rng, (batch, 2, 256))),
        "k_cache": _bf16_bits(_normal(rng, (batch, max_ctx, 2, 256))),
        "v_cache": _bf16_bits(_normal(rng, (batch, max_ctx, 2, 256))),
    }


def q4_weight(rows: int, cols: int, seed: int, sb_dtype: str = "f16"):
    """MLX affine Q4, group 64: w uint32 [rows, cols/8] of random nibbles,
    scales ~U(0.005, 0.02) and biases ~N(0, 0.05), as f16 (or bf16) bits
    [rows, cols/64]."""
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 2 ** 32, (rows, cols // 8), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(0.005, 0.02, (rows, cols // 64)).astype(np.float32)
    b = _normal(rng, (rows, cols // 64), 0.05)
    if sb_dtype == "f16":
        return w, s.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    return w, _bf16_bits(s), _bf16_bits(b)


def q8_weight(rows: int, cols: int, seed: int, sb_dtype: str = "bf16"):
    """MLX affine Q8, group 64: w uint32 [rows, cols/4] of random bytes,
    scales ~U(0.001, 0.004) and biases ~N(0, 0.1), as bf16 (or f16) bits
    [rows, cols/64]."""
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 2 ** 32, (rows, cols // 4), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(0.001, 0.004, (rows, cols // 64)).astype(np.float32)
    b = _normal(rng, (rows, cols // 64), 0.1)
    if sb_dtype == "f16":
        return w, s.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    return w, _bf16_bits(s), _bf16_bits(b)
