"""numpy front-end to the C oracle (oracle/qff_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker, never as the product.

Each wrapper names the reference lines its C function restates. Arrays are
numpy; dtype codes follow include/qff/qff.h (0 f32, 1 bf16, 2 f16), with bf16
and f16 carried as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libqff_oracle.so")

F32, BF16, F16 = 0, 1, 2

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc, no reference sources)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)
_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_d = ctypes.c_double


def _declare(L):
    for sfx, P, S in (("_f32", _fp, _f), ("_f64", _dp, _d)):
        getattr(L, "qffo_silu" + sfx).restype = S
        getattr(L, "qffo_silu" + sfx).argtypes = [S]
        getattr(L, "qffo_sigmoid" + sfx).restype = S
        getattr(L, "qffo_sigmoid" + sfx).argtypes = [S]
        getattr(L, "qffo_softplus" + sfx).restype = S
        getattr(L, "qffo_softplus" + sfx).argtypes = [S]
        getattr(L, "qffo_rmsnorm" + sfx).argtypes = [P, P, _i, S, _i, P]
        getattr(L, "qffo_matvec" + sfx).argtypes = [P, P, _i, _i, P]
        getattr(L, "qffo_conv1d_step" + sfx).argtypes = [P, P, P, _i, P]
        getattr(L, "qffo_l2norm" + sfx).argtypes = [P, _i, S, P]
        getattr(L, "qffo_deltanet_recurrent_step" + sfx).argtypes = [P] * 9
        getattr(L, "qffo_gated_rmsnorm" + sfx).argtypes = [P, P, P, S, P]
        getattr(L, "qffo_deltanet_token" + sfx).argtypes = [P] * 8 + [S, P, P, P]
        getattr(L, "qffo_deltanet_sequence" + sfx).argtypes = [_i] + [P] * 8 + [S, P, P, P]
        getattr(L, "qffo_head_rmsnorm" + sfx).argtypes = [P, P, _i, _i, S]
        getattr(L, "qffo_rope_tables" + sfx).argtypes = [_i, S, _i, P, P]
        getattr(L, "qffo_rope_partial" + sfx).argtypes = [P, P, P, _i, _i, _i]
        getattr(L, "qffo_attention_decode" + sfx).argtypes = [P, P, P, _i, _i, _i, _i, S, _i, P]
        getattr(L, "qffo_q4_matvec" + sfx).argtypes = [_vp, P, P, P, _i, _i, P]
    L.qffo_f32_to_bf16.restype = ctypes.c_uint16
    L.qffo_f32_to_bf16.argtypes = [_f]
    L.qffo_bf16_to_f32.restype = _f
    L.qffo_bf16_to_f32.argtypes = [ctypes.c_uint16]
    L.qffo_f32_to_f16.restype = ctypes.c_uint16
    L.qffo_f32_to_f16.argtypes = [_f]
    L.qffo_f16_to_f32.restype = _f
    L.qffo_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.qffo_round_to.restype = _f
    L.qffo_round_to.argtypes = [_f, _i]
    L.qffo_q4_dequant.argtypes = [_vp, _vp, _vp, _i, _i, _i, _fp]
    L.qffo_q8_dequant.argtypes = [_vp, _vp, _vp, _i, _i, _i, _fp]
    L.qffo_router_logits.argtypes = [_vp, _vp, _vp, _i, _fp, _i, _i, _fp]
    L.qffo_router_top8.argtypes = [_fp, _i, _vp, _fp]
    L.qffo_kv_append.argtypes = [_fp, _fp, _vp, _vp, _i, _i, _i, _i, _i]
    L.qffo_attention_gate.argtypes = [_vp, _fp, _i, _fp]
    L.qffo_gqa_append_kv.argtypes = [_fp, _fp, _fp, _f, _i, _f, _vp, _vp, _i, _i, _i]
    L.qffo_gqa_append_kv_seq.argtypes = [_i, _i, _fp, _fp, _fp, _f, _i, _f, _vp, _vp, _i, _i]
    L.qffo_gqa_attend.argtypes = [_fp, _fp, _f, _i, _f, _f, _vp, _vp, _i, _i, _i, _i, _i, _fp]
    L.qffo_gqa_attend_f64.argtypes = [_dp, _dp, _d, _i, _d, _d, _vp, _vp, _i, _i, _dp]


def _real(prec):
    return (np.float32, _fp, "_f32") if prec == 32 else (np.float64, _dp, "_f64")


def _arr(x, dt):
    return np.ascontiguousarray(x, dtype=dt)


def _p(a, P):
    return a.ctypes.data_as(P)


# ---------------------------------------------------------------- dtypes
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """RNE float32 -> bf16 bits (vectorised; agrees with qffo_f32_to_bf16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_to_f32(f32_to_bf16(x))


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_to_f32(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def to_real(x, dtype_code):
    """Stored bits (uint16) or f32 -> float32 values."""
    if dtype_code == BF16:
        return bf16_to_f32(x)
    if dtype_code == F16:
        return f16_to_f32(x)
    return np.asarray(x, dtype=np.float32)


# ---------------------------------------------------------------- scalars
def silu(x, prec=32):
    return getattr(lib(), "qffo_silu" + _real(prec)[2])(x)


def sigmoid(x, prec=32):
    return getattr(lib(), "qffo_sigmoid" + _real(prec)[2])(x)


def softplus(x, prec=32):
    return getattr(lib(), "qffo_softplus" + _real(prec)[2])(x)


# ---------------------------------------------------------------- DeltaNet
def rmsnorm(x, w, eps=1e-6, one_plus_w=False, prec=32):
    """QwenDeltaNetKernel.swift:22-37 (one_plus_w) / deltanet.metal:18-53."""
    dt, P, s = _real(prec)
    x, w = _arr(x, dt), _arr(w, dt)
    out = np.empty_like(x)
    getattr(lib(), "qffo_rmsnorm" + s)(_p(x, P), _p(w, P), x.size, eps, int(one_plus_w), _p(out, P))
    return out


def matvec(w, x, prec=32):
    """QwenDeltaNetKernel.swift:153-167."""
    dt, P, s = _real(prec)
    w, x = _arr(w, dt), _arr(x, dt)
    rows, cols = w.shape
    y = np.empty(rows, dt)
    getattr(lib(), "qffo_matvec" + s)(_p(w, P), _p(x, P), rows, cols, _p(y, P))
    return y


def conv1d_step(x, state, w, prec=32):
    """QwenDeltaNetKernel.swift:39-59. Returns (out, new_state)."""
    dt, P, s = _real(prec)
    x, w = _arr(x, dt), _arr(w, dt)
    st = _arr(state, dt).copy()
    out = np.empty_like(x)
    getattr(lib(), "qffo_conv1d_step" + s)(_p(x, P), _p(st, P), _p(w, P), x.size, _p(out, P))
    return out, st


def l2norm(v, eps=1e-6, prec=32):
    """QwenDeltaNetKernel.swift:61-71."""
    dt, P, s = _real(prec)
    v = _arr(v, dt)
    out = np.empty_like(v)
    getattr(lib(), "qffo_l2norm" + s)(_p(v, P), v.size, eps, _p(out, P))
    return out


def deltanet_recurrent_step(q, k, v, a, b, a_log, dt_bias, state, prec=32):
    """QwenDeltaNetKernel.swift:73-125. q,k,v [32,128]; state [32,128,128]."""
    dt, P, s = _real(prec)
    args = [_arr(x, dt) for x in (q, k, v, a, b, a_log, dt_bias)]
    st = _arr(state, dt).copy()
    out = np.empty((32, 128), dt)
    getattr(lib(), "qffo_deltanet_recurrent_step" + s)(*[_p(x, P) for x in args], _p(st, P), _p(out, P))
    return out, st


def gated_rmsnorm(core, w, z, eps=1e-6, prec=32):
    """QwenDeltaNetKernel.swift:127-151."""
    dt, P, s = _real(prec)
    core, w, z = _arr(core, dt), _arr(w, dt), _arr(z, dt)
    out = np.empty(4096, dt)
    getattr(lib(), "qffo_gated_rmsnorm" + s)(_p(core, P), _p(w, P), _p(z, P), eps, _p(out, P))
    return out


def deltanet_sequence(qkv, z, a, b, a_log, dt_bias, conv_w, norm_w, conv_state,
                      ssm_state, eps=1e-6, prec=32):
    """T tokens through the layer core one at a time (QwenDeltaNetKernel.swift
    :178-255 steps 3-6, fed token by token as QwenQ4ActiveExpertStreamingRunner
    .swift:1545-1561 does). qkv [T,8192] (pre-conv), z [T,4096], a,b [T,32],
    conv_state [8192,4], ssm_state [32,128,128]. Returns (out [T,4096],
    conv_state, ssm_state)."""
    dt, P, s = _real(prec)
    qkv = _arr(qkv, dt).reshape(-1, 8192)
    T = qkv.shape[0]
    z = _arr(z, dt).reshape(T, 4096)
    a = _arr(a, dt).reshape(T, 32)
    b = _arr(b, dt).reshape(T, 32)
    prm = [_arr(x, dt) for x in (a_log, dt_bias, conv_w, norm_w)]
    cs = _arr(conv_state, dt).reshape(8192, 4).copy()
    ss = _arr(ssm_state, dt).reshape(32, 128, 128).copy()
    out = np.empty((T, 4096), dt)
    getattr(lib(), "qffo_deltanet_sequence" + s)(
        T, _p(qkv, P), _p(z, P), _p(a, P), _p(b, P), *[_p(x, P) for x in prm],
        eps, _p(cs, P), _p(ss, P), _p(out, P))
    return out, cs, ss


# ---------------------------------------------------------------- GQA
def head_rmsnorm(x, w, eps=1e-6, prec=32):
    """deltanet.metal:614-632. x [nheads, hd]."""
    dt, P, s = _real(prec)
    x = _arr(x, dt).copy()
    w = _arr(w, dt)
    nh, hd = x.shape
    getattr(lib(), "qffo_head_rmsnorm" + s)(_p(x, P), _p(w, P), nh, hd, eps)
    return x


def rope_tables(pos, theta=1e7, rot=64, prec=32):
    """QwenQ4ActiveExpertStreamingRunner.swift:1090-1099."""
    dt, P, s = _real(prec)
    c = np.empty(rot, dt)
    sn = np.empty(rot, dt)
    getattr(lib(), "qffo_rope_tables" + s)(pos, theta, rot, _p(c, P), _p(sn, P))
    return c, sn


def rope_partial(x, cos_t, sin_t, rot=64, prec=32):
    """deltanet.metal:634-651. x [nheads, hd]."""
    dt, P, s = _real(prec)
    x = _arr(x, dt).copy()
    c, sn = _arr(cos_t, dt), _arr(sin_t, dt)
    nh, hd = x.shape
    getattr(lib(), "qffo_rope_partial" + s)(_p(x, P), _p(c, P), _p(sn, P), nh, hd, rot)
    return x


def attention_decode(q, K, V, scale=1.0 / 16, num_chunks=0, prec=32):
    """attention.metal:134-377 with Attention.swift:129-157 geometry
    (num_chunks=0) or a forced chunk count. q [nq,hd]; K,V [L,nkv,hd]."""
    dt, P, s = _real(prec)
    q, K, V = _arr(q, dt), _arr(K, dt), _arr(V, dt)
    nq, hd = q.shape
    L, nkv, _ = K.shape
    out = np.empty((nq, hd), dt)
    getattr(lib(), "qffo_attention_decode" + s)(_p(q, P), _p(K, P), _p(V, P), L, nq, nkv, hd,
                                                scale, num_chunks, _p(out, P))
    return out


def kv_append(k, v, k_cache, v_cache, cache_dtype, pos):
    """deltanet.metal:670-689 into caches [max_seq, nkv, hd] (uint16 bits for
    bf16/f16). Caches are updated in place."""
    k, v = _arr(k, np.float32), _arr(v, np.float32)
    max_seq, nkv, hd = k_cache.shape
    lib().qffo_kv_append(_p(k, _fp), _p(v, _fp), k_cache.ctypes.data, v_cache.ctypes.data,
                         cache_dtype, pos, max_seq, nkv, hd)


def attention_gate(attn_half_bits, gate):
    """deltanet.metal:700-708."""
    a = np.ascontiguousarray(attn_half_bits, dtype=np.uint16)
    g = _arr(gate, np.float32)
    out = np.empty(g.size, np.float32)
    lib().qffo_attention_gate(a.ctypes.data, _p(g, _fp), g.size, _p(out, _fp))
    return out


def gqa_append_kv_seq(k, v, k_norm_w, k_cache, v_cache, cache_dtype, start_pos=0,
                      theta=1e7, rot=64, eps=1e-6):
    """k, v [T,2,256] raw projections; caches [max_seq,2,256] updated in place:
    head RMSNorm + RoPE of k at positions start_pos.., then the append."""
    k = _arr(k, np.float32).reshape(-1, 512)
    v = _arr(v, np.float32).reshape(-1, 512)
    w = _arr(k_norm_w, np.float32)
    max_seq = k_cache.shape[0]
    lib().qffo_gqa_append_kv_seq(k.shape[0], start_pos, _p(k, _fp), _p(v, _fp), _p(w, _fp),
                                 theta, rot, eps, k_cache.ctypes.data, v_cache.ctypes.data,
                                 cache_dtype, max_seq)


def gqa_attend(q_gate, q_norm_w, k_cache, v_cache, cache_dtype, pos, theta=1e7, rot=64,
               scale=1.0 / 16, eps=1e-6, q_dtype=F16, attn_dtype=F16, num_chunks=0):
    """One query token at `pos` against cache entries 0..pos, reference order.
    q_gate [16,512]. Returns out [16,256] f32."""
    qg = _arr(q_gate, np.float32)
    w = _arr(q_norm_w, np.float32)
    out = np.empty((16, 256), np.float32)
    lib().qffo_gqa_attend(_p(qg, _fp), _p(w, _fp), theta, rot, scale, eps,
                          k_cache.ctypes.data, v_cache.ctypes.data, cache_dtype, pos,
                          q_dtype, attn_dtype, num_chunks, _p(out, _fp))
    return out


def gqa_attend_f64(q_gate, q_norm_w, k_cache, v_cache, cache_dtype, pos, theta=1e7,
                   rot=64, scale=1.0 / 16, eps=1e-6):
    qg = _arr(q_gate, np.float64)
    w = _arr(q_norm_w, np.float64)
    out = np.empty((16, 256), np.float64)
    lib().qffo_gqa_attend_f64(_p(qg, _dp), _p(w, _dp), theta, rot, scale, eps,
                              k_cache.ctypes.data, v_cache.ctypes.data, cache_dtype, pos,
                              _p(out, _dp))
    return out


# ---------------------------------------------------------------- Q4
def q4_dequant(w, scales, biases, sb_dtype=F16):
    """QwenQ4ActiveExpertStreamingRunner.swift:899-922 closed form.
    w uint32 [rows, cols/8]; scales/biases uint16 bits [rows, cols/64]."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    rows, c8 = w.shape
    cols = c8 * 8
    s = np.ascontiguousarray(scales)
    b = np.ascontiguousarray(biases)
    out = np.empty((rows, cols), np.float32)
    lib().qffo_q4_dequant(w.ctypes.data, s.ctypes.data, b.ctypes.data, sb_dtype, rows, cols,
                          _p(out, _fp))
    return out


def q4_matvec(w, scales, biases, x, sb_dtype=F16, prec=32):
    """deltanet.metal:816-861 factored order. x [cols] -> y [rows]."""
    dt, P, s = _real(prec)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    rows, c8 = w.shape
    cols = c8 * 8
    sc = _arr(to_real(scales, sb_dtype), dt)
    bi = _arr(to_real(biases, sb_dtype), dt)
    x = _arr(x, dt)
    y = np.empty(rows, dt)
    getattr(lib(), "qffo_q4_matvec" + s)(w.ctypes.data, _p(sc, P), _p(bi, P), _p(x, P), rows,
                                         cols, _p(y, P))
    return y


def q8_dequant(w, scales, biases, sb_dtype=BF16):
    """deltanet.metal:863-900 closed form. w uint32 [rows, cols/4] (byte c of
    a row = element c); scales/biases uint16 bits [rows, cols/64]."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    rows, c4 = w.shape
    cols = c4 * 4
    s = np.ascontiguousarray(scales)
    b = np.ascontiguousarray(biases)
    out = np.empty((rows, cols), np.float32)
    lib().qffo_q8_dequant(w.ctypes.data, s.ctypes.data, b.ctypes.data, sb_dtype, rows, cols, _p(out, _fp))
    return out


def router_logits(w, scales, biases, x, sb_dtype=BF16):
    """deltanet.metal:2229-2259 factored order. x [cols] f32 -> [rows] f32."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    rows, c4 = w.shape
    s = np.ascontiguousarray(scales)
    b = np.ascontiguousarray(biases)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(rows, np.float32)
    lib().qffo_router_logits(w.ctypes.data, s.ctypes.data, b.ctypes.data, sb_dtype, _p(x, _fp), rows, c4 * 4,
                             _p(out, _fp))
    return out


def router_top8(logits):
    """deltanet.metal:2283-2329: (indices int32 [8], scores f32 [8])."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.empty(8, np.int32)
    sc = np.empty(8, np.float32)
    lib().qffo_router_top8(_p(lg, _fp), lg.size, idx.ctypes.data, _p(sc, _fp))
    return idx, sc
