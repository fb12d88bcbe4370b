"""numpy front-end to oracle/cpu_baseline.c: the reference's CPU algorithms
with OpenMP drivers, timed as bench.py's CPU baseline.

TEST INFRASTRUCTURE ONLY: loaded by bench.py's cpu_baseline leg and by
tests/ (which check it against the oracle bit for bit), never by the
product.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PORTABLE = os.path.join(HERE, "build", "libqff_cpu_baseline.so")
NATIVE_FLAGS = ["-O3", "-march=native", "-fopenmp", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-std=c11"]

_fp = ctypes.POINTER(ctypes.c_float)


def build_native(outdir: str) -> str | None:
    """Compile cpu_baseline.c for the host this runs on (gcc -O3
    -march=native -fopenmp) into outdir; None when no compiler works."""
    os.makedirs(outdir, exist_ok=True)
    out = os.path.join(outdir, "libqff_cpu_baseline_native.so")
    cmd = ["gcc", *NATIVE_FLAGS, "-shared", "-o", out, os.path.join(HERE, "cpu_baseline.c"), "-lm"]
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    except (OSError, subprocess.SubprocessError):
        return None
    return out if r.returncode == 0 else None


def load(path: str | None = None):
    L = ctypes.CDLL(path or PORTABLE)
    L.qffb_openmp.restype = ctypes.c_int
    L.qffb_deltanet_prefill.argtypes = [ctypes.c_int] + [_fp] * 8 + [ctypes.c_float] + [_fp] * 4 + [ctypes.c_int]
    L.qffb_attention_decode.argtypes = [ctypes.c_int, _fp, _fp, _fp, ctypes.c_void_p, ctypes.c_int,
                                        ctypes.c_float, _fp, ctypes.c_int]
    _u = ctypes.c_void_p
    L.qffb_gqa_prefill_tokens.argtypes = ([ctypes.c_int, ctypes.c_int, _fp, _u, _fp, _fp, _fp, _fp]
                                          + [ctypes.c_float] * 3 + [_fp] * 3 + [ctypes.c_int])
    L.qffb_dn_layer_decode.argtypes = ([ctypes.c_int, _fp, _fp, _u, _fp, _fp, _u, _fp, _fp] + [_fp] * 4
                                       + [ctypes.c_float, _fp, _fp, ctypes.c_int])
    L.qffb_gqa_layer_decode.argtypes = ([ctypes.c_int, _fp, _fp, _u, _fp, _fp, _u, _fp, _fp, _fp, _fp]
                                        + [ctypes.c_float] * 3 + [_fp, _fp, _u, ctypes.c_int, ctypes.c_int])
    return L


def _f(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return a.ctypes.data_as(_fp)


def deltanet_prefill(L, qkv, z, a, b, prm, conv_state, ssm_state, threads=1, eps=1e-6):
    """T tokens through the DeltaNet layer core (QwenDeltaNetKernel.swift
    :39-151 token by token). Returns (out [T,4096], conv_state, ssm_state)."""
    qkv = _f(qkv).reshape(-1, 8192)
    T = qkv.shape[0]
    z, a, b = _f(z).reshape(T, 4096), _f(a).reshape(T, 32), _f(b).reshape(T, 32)
    pr = [_f(prm[k]) for k in ("a_log", "dt_bias", "conv_w", "norm_w")]
    cs = _f(conv_state).reshape(8192, 4).copy()
    ss = _f(ssm_state).reshape(32, 128, 128).copy()
    out = np.empty((T, 4096), np.float32)
    work = np.empty((T, 8192), np.float32)
    L.qffb_deltanet_prefill(T, _p(qkv), _p(z), _p(a), _p(b), *[_p(x) for x in pr], eps, _p(cs), _p(ss),
                            _p(out), _p(work), threads)
    return out, cs, ss


def attention_decode(L, q, K, V, lengths, scale=1.0 / 16, threads=1):
    """Split-KV decode attention (attention.metal:134-224, 342-377) of B
    sequences: q [B,16,256], K, V [B,max_ctx,2,256] fp32, lengths [B] ->
    out [B,16,256]."""
    q, K, V = _f(q), _f(K), _f(V)
    B, max_ctx = K.shape[0], K.shape[1]
    lens = np.ascontiguousarray(lengths, dtype=np.int32)
    out = np.empty((B, 16, 256), np.float32)
    L.qffb_attention_decode(B, _p(q), _p(K), _p(V), lens.ctypes.data, max_ctx, scale, _p(out), threads)
    return out


def q4_stack(parts):
    """Affine-Q4 parts (w uint32 [rows, cols/8], scales, biases as fp32
    reals [rows, cols/64]) stacked along rows into one weight, as the
    drivers take the grouped projections."""
    w = np.ascontiguousarray(np.concatenate([p[0] for p in parts]), dtype=np.uint32)
    sc = _f(np.concatenate([p[1] for p in parts]))
    bi = _f(np.concatenate([p[2] for p in parts]))
    return w, sc, bi


def gqa_prefill_tokens(L, t0, t1, x, w, sc, bi, q_norm_w, k_norm_w, K, V, out, theta=1e7, scale=1.0 / 16,
                       eps=1e-6, threads=1):
    """Tokens t0 .. t1-1 of one sequence through the full-attention core,
    token by token (the reference's prefill): x [T, 2048]; (w, sc, bi) the
    9216-row q|gate, k, v weight (q4_stack); K, V [max_ctx, 2, 256] fp32
    caches and out [T, 16, 256] updated in place."""
    L.qffb_gqa_prefill_tokens(t0, t1, _p(x), w.ctypes.data, _p(sc), _p(bi), _p(_f(q_norm_w)), _p(_f(k_norm_w)),
                              theta, scale, eps, _p(K), _p(V), _p(out), threads)


def dn_layer_decode(L, x, in_norm_w, w_in, w_out, prm, conv_state, ssm, eps=1e-6, threads=1):
    """B decode tokens through one Gated DeltaNet layer's attention block
    (x [B, 2048], conv_state [B, 8192, 4], ssm [B, 32, 128, 128] updated in
    place); w_in the stacked 12352-row in-projection, w_out the 2048 x 4096
    out-projection, each (w, scales, biases) as q4_stack returns."""
    pr = [_p(_f(prm[k])) for k in ("a_log", "dt_bias", "conv_w", "norm_w")]
    L.qffb_dn_layer_decode(x.shape[0], _p(x), _p(_f(in_norm_w)), w_in[0].ctypes.data, _p(w_in[1]), _p(w_in[2]),
                           w_out[0].ctypes.data, _p(w_out[1]), _p(w_out[2]), *pr, eps, _p(conv_state), _p(ssm),
                           threads)


def gqa_layer_decode(L, x, in_norm_w, w_in, w_out, q_norm_w, k_norm_w, K, V, positions, theta=1e7,
                     scale=1.0 / 16, eps=1e-6, threads=1):
    """B decode tokens through one full-attention layer's attention block:
    x [B, 2048] updated in place; K, V [B, max_ctx, 2, 256] fp32 caches
    appended at positions [B]."""
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    L.qffb_gqa_layer_decode(x.shape[0], _p(x), _p(_f(in_norm_w)), w_in[0].ctypes.data, _p(w_in[1]), _p(w_in[2]),
                            w_out[0].ctypes.data, _p(w_out[1]), _p(w_out[2]), _p(_f(q_norm_w)), _p(_f(k_norm_w)),
                            theta, scale, eps, _p(K), _p(V), pos.ctypes.data, K.shape[1], threads)
