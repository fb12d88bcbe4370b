"""One decoder layer's attention block on the CPU oracle, in the reference's
encoder order (QwenQ4ActiveExpertStreamingRunner.swift:972-1040 for a Gated
DeltaNet layer, :1041-1167 for a full-attention layer), for one sequence:

  x' = x + out_proj(core(in_proj(rmsnorm(x, in_norm_w))))

The Q4 products use the oracle's factored fp32 order (deltanet.metal
:1838-1895), the input RMSNorm weights as they are (deltanet.metal:18-53),
the DeltaNet core the sequential fp32 recurrence (QwenDeltaNetKernel.swift
:39-151) and the full-attention core the reference's split / head norms /
RoPE / append / fp16 q / split-KV attention / gate (oracle gqa_*)."""
import numpy as np
import torch

from oracle import oracle as O


def _np(t):
    if isinstance(t, np.ndarray):
        return t
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return O.bf16_to_f32(t.view(torch.int16).numpy().view(np.uint16))
    return t.float().numpy()


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def q4_part_np(part):
    """(w uint32, scales bits, biases bits, sb dtype code) of a device Q4 part."""
    w, s, b = part
    code = O.F16 if s.dtype == torch.float16 else O.BF16
    return w.detach().cpu().numpy().view(np.uint32), _bits(s), _bits(b), code


def q4_mv(part_np, x):
    w, s, b, code = part_np
    return O.q4_matvec(w, s, b, x.astype(np.float32), code)


def deltanet_layer(layer_np, x, conv, ssm, eps=1e-6):
    """layer_np: {"in_norm_w", "in_proj": 4 parts (qkv, z, b, a), "out_proj",
    "params"} as numpy. Returns (x', conv', ssm')."""
    xn = O.rmsnorm(x, layer_np["in_norm_w"], eps)
    qkv, z, bb, aa = (q4_mv(p, xn) for p in layer_np["in_proj"])
    p = layer_np["params"]
    out, cs, ss = O.deltanet_sequence(qkv[None], z[None], aa[None], bb[None], p["a_log"], p["dt_bias"],
                                      p["conv_w"], p["norm_w"], conv, ssm, eps=eps)
    return x + q4_mv(layer_np["out_proj"], out[0]), cs, ss


def gqa_layer(layer_np, x, k_cache, v_cache, pos, eps=1e-6):
    """layer_np: {"in_norm_w", "in_proj": 3 parts (q|gate, k, v), "out_proj",
    "params"}; caches [max_ctx, 2, 256] bf16 bits, updated in place at pos.
    Returns x'."""
    xn = O.rmsnorm(x, layer_np["in_norm_w"], eps)
    qg, k, v = (q4_mv(p, xn) for p in layer_np["in_proj"])
    p = layer_np["params"]
    O.gqa_append_kv_seq(k.reshape(1, 2, 256), v.reshape(1, 2, 256), p["k_norm_w"], k_cache, v_cache, O.BF16,
                        start_pos=pos, eps=eps)
    att = O.gqa_attend(qg.reshape(16, 512), p["q_norm_w"], k_cache, v_cache, O.BF16, pos, eps=eps)
    return x + q4_mv(layer_np["out_proj"], att.reshape(4096))


def layer_to_np(layer):
    """A device layer dict (Checkpoint.deltanet_layer / gqa_layer layout) to
    the numpy form above."""
    return {"in_norm_w": _np(layer["in_norm_w"]),
            "in_proj": [q4_part_np(p) for p in layer["in_proj"]],
            "out_proj": q4_part_np(layer["out_proj"]),
            "params": {k: _np(v) for k, v in layer["params"].items()}}
