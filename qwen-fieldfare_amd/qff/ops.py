"""torch-facing wrappers over the C ABI.

Each wrapper mirrors one encoder block of the reference's per-layer schedule
(QwenQ4ActiveExpertStreamingRunner.swift:972-1167): it checks the tensors it
is handed, passes their device pointers and torch's current stream to the
library, and raises QffError on any non-zero status. Outputs are allocated
here only when the caller does not pass them.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import BF16, F16, F32, Q4_MAX_PARTS, CtxCfg, DeltaNetParams, GqaParams, Q4Part, QffError, check, lib

_DT = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}
_TORCH = {F32: torch.float32, BF16: torch.bfloat16, F16: torch.float16}


def _code(t: torch.Tensor) -> int:
    if t.dtype not in _DT:
        raise TypeError(f"unsupported dtype {t.dtype}")
    return _DT[t.dtype]


def _ptr(t: torch.Tensor):
    if not t.is_cuda:
        raise ValueError("tensor must live on the GPU")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class Context:
    """Owns a qff_ctx: the device workspace for the hot calls (replaces the
    reference's MetalContext + Attention scratch set-up)."""

    def __init__(self, device: int = 0, max_batch: int = 32, max_ctx: int = 65536,
                 max_prefill_tokens: int = 8192):
        self.device = device
        h = ctypes.c_void_p()
        cfg = CtxCfg(max_batch, max_ctx, max_prefill_tokens)
        check("qff_ctx_create", lib().qff_ctx_create(ctypes.byref(h), device, ctypes.byref(cfg)))
        self.handle = h
        self.cfg = cfg

    def close(self):
        if self.handle:
            check("qff_ctx_destroy", lib().qff_ctx_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def q4_dequant(ctx: Context, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """w int32/uint32 [rows, cols/8]; scales/biases f16/bf16 [rows, cols/64] -> f32 [rows, cols]."""
    rows, c8 = w.shape
    if out is None:
        out = torch.empty(rows, c8 * 8, dtype=torch.float32, device=w.device)
    check("qff_q4_dequant", lib().qff_q4_dequant(ctx.handle, _stream(), _ptr(w), _ptr(scales),
                                                 _ptr(biases), _code(scales), _ptr(out), rows, c8 * 8))
    return out


def q4_matmul(ctx: Context, w, scales, biases, x: torch.Tensor, out=None,
              out_dtype=torch.float32) -> torch.Tensor:
    """x [batch, cols] (f32/bf16) -> y [batch, rows]."""
    rows, c8 = w.shape
    cols = c8 * 8
    x2 = x.reshape(-1, cols)
    batch = x2.shape[0]
    if out is None:
        out = torch.empty(batch, rows, dtype=out_dtype, device=x.device)
    check("qff_q4_matmul", lib().qff_q4_matmul(ctx.handle, _stream(), _ptr(w), _ptr(scales),
                                               _ptr(biases), _code(scales), _ptr(x2), _code(x2),
                                               _ptr(out), _code(out), rows, cols, batch))
    return out


def _q4_parts(parts, x, outs, out_dtypes, residuals):
    if not 1 <= len(parts) <= Q4_MAX_PARTS:
        raise ValueError(f"1 .. {Q4_MAX_PARTS} parts")
    cols = parts[0][0].shape[1] * 8
    x2 = x.reshape(-1, cols)
    batch = x2.shape[0]
    arr = (Q4Part * len(parts))()
    res = []
    for i, (w, s, b) in enumerate(parts):
        rows = w.shape[0]
        if w.shape[1] * 8 != cols or s.dtype != parts[0][1].dtype:
            raise ValueError("parts must share cols and scale dtype")
        if outs is not None:
            out = outs[i]
        else:
            dt = out_dtypes[i] if out_dtypes is not None else torch.float32
            out = torch.empty(batch, rows, dtype=dt, device=x.device)
        r = residuals[i] if residuals is not None else None
        if r is not None and (r.dtype != out.dtype or r.numel() != out.numel()):
            raise ValueError("a residual must match its output's dtype and size")
        arr[i] = Q4Part(_ptr(w), _ptr(s), _ptr(b), rows, _ptr(out), _code(out), _ptr(r) if r is not None else None)
        res.append(out)
    return arr, res, x2, cols, batch


def q4_matmul_parts(ctx: Context, parts, x: torch.Tensor, outs=None, out_dtypes=None, residuals=None):
    """One launch of y_p = x W_p^T (+ residual_p) for every part (w, scales,
    biases) in `parts` (all with the same cols and scale dtype), sharing x
    [batch, cols]. `residuals`: per part None or a tensor of the output's
    dtype and shape (may be the output itself). Returns the outputs
    [batch, rows_p]."""
    arr, res, x2, cols, batch = _q4_parts(parts, x, outs, out_dtypes, residuals)
    check("qff_q4_matmul_parts", lib().qff_q4_matmul_parts(ctx.handle, _stream(), arr, len(parts),
                                                           _code(parts[0][1]), _ptr(x2), _code(x2), cols, batch))
    return res


def q4_norm_matmul_parts(ctx: Context, parts, x: torch.Tensor, norm_w: torch.Tensor, eps: float = 1e-6,
                         outs=None, out_dtypes=None, residuals=None):
    """The layer front-end: RMSNorm of each token of x (weight norm_w [cols],
    f32 or bf16, eps) feeding the grouped product of q4_matmul_parts."""
    arr, res, x2, cols, batch = _q4_parts(parts, x, outs, out_dtypes, residuals)
    if norm_w.numel() != cols:
        raise ValueError("norm_w must have cols entries")
    check("qff_q4_norm_matmul_parts", lib().qff_q4_norm_matmul_parts(
        ctx.handle, _stream(), arr, len(parts), _code(parts[0][1]), _ptr(x2), _code(x2), _ptr(norm_w),
        _code(norm_w), eps, cols, batch))
    return res


def q8_dequant(ctx: Context, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """w int32/uint32 [rows, cols/4]; scales/biases bf16/f16 [rows, cols/64] -> f32 [rows, cols]."""
    rows, c4 = w.shape
    if out is None:
        out = torch.empty(rows, c4 * 4, dtype=torch.float32, device=w.device)
    check("qff_q8_dequant", lib().qff_q8_dequant(ctx.handle, _stream(), _ptr(w), _ptr(scales),
                                                 _ptr(biases), _code(scales), _ptr(out), rows, c4 * 4))
    return out


def router_top8(ctx: Context, w, scales, biases, x: torch.Tensor, logits=None, indices=None, scores=None):
    """MoE router: Q8 logits of x [batch, cols] over the experts (rows of
    w), then the top eight per token. Returns (indices int32 [batch, 8],
    scores f32 [batch, 8], logits f32 [batch, experts])."""
    experts, c4 = w.shape
    cols = c4 * 4
    x2 = x.reshape(-1, cols)
    batch = x2.shape[0]
    dev = x.device
    if logits is None:
        logits = torch.empty(batch, experts, dtype=torch.float32, device=dev)
    if indices is None:
        indices = torch.empty(batch, 8, dtype=torch.int32, device=dev)
    if scores is None:
        scores = torch.empty(batch, 8, dtype=torch.float32, device=dev)
    check("qff_router_top8", lib().qff_router_top8(ctx.handle, _stream(), _ptr(w), _ptr(scales), _ptr(biases),
                                                   _code(scales), _ptr(x2), _code(x2), _ptr(logits), _ptr(indices),
                                                   _ptr(scores), experts, cols, batch))
    return indices, scores, logits


def _dn_params(p: dict, eps: float):
    for k in ("a_log", "dt_bias", "conv_w", "norm_w"):
        if p[k].dtype != torch.float32:
            raise TypeError(f"{k} must be float32")
    return DeltaNetParams(_ptr(p["a_log"]), _ptr(p["dt_bias"]), _ptr(p["conv_w"]), _ptr(p["norm_w"]), eps)


def _check_dn_inputs(qkv, z, a, b, conv_state, ssm_state, n, seqs):
    """n tokens of `seqs` sequences: the shapes and element types the
    library assumes, checked before any pointer reaches it."""
    if z.dtype != qkv.dtype:
        raise TypeError("qkv and z must share a dtype")
    for name, t in (("a", a), ("b", b), ("conv_state", conv_state), ("ssm_state", ssm_state)):
        if t.dtype != torch.float32:
            raise TypeError(f"{name} must be float32")
    if qkv.numel() != n * 8192 or z.numel() != n * 4096 or a.numel() != n * 32 or b.numel() != n * 32:
        raise ValueError("qkv, z, a, b must be [n, 8192], [n, 4096], [n, 32], [n, 32]")
    if conv_state.numel() != seqs * 8192 * 4 or ssm_state.numel() != seqs * 32 * 128 * 128:
        raise ValueError("conv_state / ssm_state must hold [8192, 4] / [32, 128, 128] per sequence")


def deltanet_decode(ctx: Context, params: dict, qkv, z, a, b, conv_state, ssm_state, out=None,
                    out_dtype=torch.bfloat16, eps: float = 1e-6) -> torch.Tensor:
    """One decode step for batch B. qkv [B,8192], z [B,4096] (same dtype), a, b
    [B,32] f32, conv_state [B,8192,4] f32, ssm_state [B,32,128,128] f32 (both
    updated in place) -> out [B,4096]."""
    B = qkv.shape[0]
    _check_dn_inputs(qkv, z, a, b, conv_state, ssm_state, B, B)
    if out is None:
        out = torch.empty(B, 4096, dtype=out_dtype, device=qkv.device)
    prm = _dn_params(params, eps)
    check("qff_deltanet_decode", lib().qff_deltanet_decode(
        ctx.handle, _stream(), ctypes.byref(prm), _ptr(qkv), _ptr(z), _code(qkv), _ptr(a), _ptr(b),
        _ptr(conv_state), _ptr(ssm_state), _ptr(out), _code(out), B))
    return out


def deltanet_prefill(ctx: Context, params: dict, qkv, z, a, b, conv_state, ssm_state, out=None,
                     out_dtype=torch.bfloat16, eps: float = 1e-6, chunk: int = 64) -> torch.Tensor:
    """T tokens of one sequence. qkv [T,8192], z [T,4096], a, b [T,32];
    conv_state [8192,4], ssm_state [32,128,128] updated in place -> out [T,4096]."""
    T = qkv.shape[0]
    _check_dn_inputs(qkv, z, a, b, conv_state, ssm_state, T, 1)
    if out is None:
        out = torch.empty(T, 4096, dtype=out_dtype, device=qkv.device)
    prm = _dn_params(params, eps)
    check("qff_deltanet_prefill", lib().qff_deltanet_prefill(
        ctx.handle, _stream(), ctypes.byref(prm), _ptr(qkv), _ptr(z), _code(qkv), _ptr(a), _ptr(b),
        _ptr(conv_state), _ptr(ssm_state), _ptr(out), _code(out), T, chunk))
    return out


def _check_gqa_inputs(q_gate, k, v, k_cache, v_cache, n):
    """The library reads q_gate, k and v with one element type and both
    caches as bf16 or both as fp16 (the reference's cache type): reject
    anything else before it reaches the device."""
    if k_cache.dtype not in (torch.bfloat16, torch.float16) or v_cache.dtype != k_cache.dtype:
        raise TypeError("KV caches must both be bfloat16 or both float16")
    if k.dtype != q_gate.dtype or v.dtype != q_gate.dtype:
        raise TypeError("k and v must share q_gate's dtype")
    if q_gate.numel() != n * 16 * 512 or k.numel() != n * 512 or v.numel() != n * 512:
        raise ValueError("q_gate must be [n, 16, 512] and k, v [n, 2, 256]")


def _gqa_params(p: dict, theta, scale, eps, k_cache):
    return GqaParams(_ptr(p["q_norm_w"]), _ptr(p["k_norm_w"]), theta, 64, scale, eps,
                     int(k_cache.dtype == torch.float16))


def gqa_decode(ctx: Context, params: dict, q_gate, k_new, v_new, k_cache, v_cache, positions,
               out=None, out_dtype=torch.bfloat16, theta=1e7, scale=1.0 / 16, eps=1e-6):
    """q_gate [B,16,512], k_new/v_new [B,2,256]; caches [B,max_ctx,2,256] bf16
    or fp16; positions int32 [B] (device) -> out [B,16,256]."""
    B = q_gate.shape[0]
    max_ctx = k_cache.shape[1]
    _check_gqa_inputs(q_gate, k_new, v_new, k_cache, v_cache, B)
    if tuple(k_cache.shape) != (B, max_ctx, 2, 256) or tuple(v_cache.shape) != tuple(k_cache.shape):
        raise ValueError("KV caches must be [B, max_ctx, 2, 256]")
    if positions.dtype != torch.int32 or positions.numel() != B:
        raise TypeError("positions must be int32 [B]")
    if out is None:
        out = torch.empty(B, 16, 256, dtype=out_dtype, device=q_gate.device)
    prm = _gqa_params(params, theta, scale, eps, k_cache)
    check("qff_gqa_decode", lib().qff_gqa_decode(
        ctx.handle, _stream(), ctypes.byref(prm), _ptr(q_gate), _ptr(k_new), _ptr(v_new),
        _code(q_gate), _ptr(k_cache), _ptr(v_cache), _ptr(positions), _ptr(out), _code(out), B,
        max_ctx))
    return out


def gqa_prefill(ctx: Context, params: dict, q_gate, k, v, k_cache, v_cache, start_pos=0, out=None,
                out_dtype=torch.bfloat16, theta=1e7, scale=1.0 / 16, eps=1e-6):
    """q_gate [T,16,512], k/v [T,2,256]; caches [max_ctx,2,256] bf16 or fp16
    -> out [T,16,256]."""
    T = q_gate.shape[0]
    max_ctx = k_cache.shape[0]
    _check_gqa_inputs(q_gate, k, v, k_cache, v_cache, T)
    if tuple(k_cache.shape) != (max_ctx, 2, 256) or tuple(v_cache.shape) != tuple(k_cache.shape):
        raise ValueError("KV caches must be [max_ctx, 2, 256]")
    if out is None:
        out = torch.empty(T, 16, 256, dtype=out_dtype, device=q_gate.device)
    prm = _gqa_params(params, theta, scale, eps, k_cache)
    check("qff_gqa_prefill", lib().qff_gqa_prefill(
        ctx.handle, _stream(), ctypes.byref(prm), _ptr(q_gate), _ptr(k), _ptr(v), _code(q_gate),
        _ptr(k_cache), _ptr(v_cache), start_pos, _ptr(out), _code(out), T, max_ctx))
    return out


__all__ = ["Context", "QffError", "q4_dequant", "q4_matmul", "deltanet_decode", "deltanet_prefill",
           "gqa_decode", "gqa_prefill", "BF16", "F16", "F32"]
