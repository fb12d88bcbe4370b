"""The attention half of the decoder stack: the per-layer schedule of
QwenQ4ActiveExpertStreamingRunner.forwardToken (Runner:924-1167) over the C
ABI, with the MoE block replaced by identity.

Layer l is full attention when l % 4 == 3, Gated DeltaNet otherwise
(Runner:554-556). Each layer reads the residual stream x [B, 2048] and adds
its attention output back into it (Runner:1034-1040, 1162-1166):

  DeltaNet   input RMSNorm + fused in-projection qkv|z|b|a (Runner:973-997)
             -> conv1d + gated delta rule + gated RMSNorm (Runner:1001-1022)
             -> out_proj, added into x (Runner:1024-1040)
  full attn  input RMSNorm + q|gate, k, v projections (Runner:1043-1074)
             -> split / head norms / RoPE / KV append / attention / gate
                (Runner:1076-1150) -> o_proj, added into x (Runner:1152-1166)

The residual stream and every intermediate are fp32, as the reference keeps
them (hiddenBuf0/1, qkvOutBuf, ... are float buffers, Runner:346-401); the KV
caches are bf16. Layers take the tensors Checkpoint.deltanet_layer /
gqa_layer return, so a stack can come from a checkpoint or from synthetic
weights of the same layout.
"""
from __future__ import annotations

import torch

from . import ops

HIDDEN = 2048


def is_full_attention(l: int) -> bool:
    return l % 4 == 3


class AttentionStack:
    """Layers, their per-sequence state and the scratch tensors of one decode
    step for `batch` sequences. `layers[l]` is a dict with the keys of
    Checkpoint.deltanet_layer (DeltaNet) or Checkpoint.gqa_layer (full
    attention); the kind follows l % 4 == 3 unless `kinds` says otherwise.
    States: DeltaNet conv [B, 8192, 4] / ssm [B, 32, 128, 128] fp32, full
    attention K / V caches [B, max_ctx, 2, 256] bf16; pass them in `states`
    or get zero states."""

    def __init__(self, ctx: ops.Context, layers, batch: int, max_ctx: int, states=None, kinds=None,
                 eps: float = 1e-6, device="cuda"):
        self.ctx = ctx
        self.layers = list(layers)
        self.B = batch
        self.max_ctx = max_ctx
        self.eps = eps
        self.kinds = list(kinds) if kinds is not None else \
            ["gqa" if is_full_attention(l) else "dn" for l in range(len(self.layers))]
        if states is None:
            states = []
            for kind in self.kinds:
                if kind == "dn":
                    states.append({"conv_state": torch.zeros(batch, 8192, 4, device=device),
                                   "ssm_state": torch.zeros(batch, 32, 128, 128, device=device)})
                else:
                    states.append({"k_cache": torch.zeros(batch, max_ctx, 2, 256, dtype=torch.bfloat16,
                                                          device=device),
                                   "v_cache": torch.zeros(batch, max_ctx, 2, 256, dtype=torch.bfloat16,
                                                          device=device)})
        self.states = states
        f32 = dict(dtype=torch.float32, device=device)
        self.qkv = torch.empty(batch, 8192, **f32)
        self.z = torch.empty(batch, 4096, **f32)
        self.a = torch.empty(batch, 32, **f32)
        self.b = torch.empty(batch, 32, **f32)
        self.core = torch.empty(batch, 4096, **f32)
        self.qg = torch.empty(batch, 8192, **f32)
        self.kn = torch.empty(batch, 512, **f32)
        self.vn = torch.empty(batch, 512, **f32)
        self.att = torch.empty(batch, 16, 256, **f32)

    def layer_step(self, l: int, x: torch.Tensor, positions: torch.Tensor):
        """Layer l of one decode step: x [B, 2048] fp32, updated in place."""
        L, S, B = self.layers[l], self.states[l], self.B
        ctx, eps = self.ctx, self.eps
        if self.kinds[l] == "dn":
            ops.q4_norm_matmul_parts(ctx, L["in_proj"], x, L["in_norm_w"], eps,
                                     outs=(self.qkv, self.z, self.b, self.a))
            ops.deltanet_decode(ctx, L["params"], self.qkv, self.z, self.a, self.b, S["conv_state"],
                                S["ssm_state"], out=self.core, eps=eps)
            ops.q4_matmul_parts(ctx, [L["out_proj"]], self.core, outs=(x,), residuals=(x,))
        else:
            ops.q4_norm_matmul_parts(ctx, L["in_proj"], x, L["in_norm_w"], eps,
                                     outs=(self.qg, self.kn, self.vn))
            ops.gqa_decode(ctx, L["params"], self.qg.view(B, 16, 512), self.kn.view(B, 2, 256),
                           self.vn.view(B, 2, 256), S["k_cache"], S["v_cache"], positions, out=self.att,
                           eps=eps)
            ops.q4_matmul_parts(ctx, [L["out_proj"]], self.att.view(B, 4096), outs=(x,), residuals=(x,))

    def decode_step(self, x: torch.Tensor, positions: torch.Tensor):
        """Every layer in order: x [B, 2048] fp32 (the residual stream, in
        place), positions int32 [B] on the device (the new token's position
        in each sequence; full-attention layers append there)."""
        if x.dtype != torch.float32 or tuple(x.shape) != (self.B, HIDDEN):
            raise ValueError(f"x must be float32 [{self.B}, {HIDDEN}]")
        for l in range(len(self.layers)):
            self.layer_step(l, x, positions)


def random_q4(rows: int, cols: int, gen: torch.Generator, device="cuda"):
    """An affine-Q4 weight with uniform nibbles, fp16 scales U(0.005, 0.02)
    and fp16 biases N(0, 0.05) (the config-3/4 distributions), made on the
    device."""
    w = torch.randint(-2 ** 31, 2 ** 31 - 1, (rows, cols // 8), dtype=torch.int32, device=device,
                      generator=gen)
    sc = (torch.rand(rows, cols // 64, device=device, generator=gen) * 0.015 + 0.005).half()
    bi = (torch.randn(rows, cols // 64, device=device, generator=gen) * 0.05).half()
    return w, sc, bi


def random_layers(n: int, gen: torch.Generator, dn_params: dict, gqa_params: dict, device="cuda"):
    """n layers of the l % 4 == 3 pattern with random affine-Q4 projections
    and input-RMSNorm weights 1; the layer constants (A_log, dt_bias, conv
    and norm weights, q/k norm weights) are shared dicts of fp32 tensors."""
    ones = torch.ones(HIDDEN, device=device)
    layers = []
    for l in range(n):
        if is_full_attention(l):
            layers.append({"in_norm_w": ones,
                           "in_proj": [random_q4(r, HIDDEN, gen, device) for r in (8192, 512, 512)],
                           "out_proj": random_q4(HIDDEN, 4096, gen, device), "params": gqa_params})
        else:
            layers.append({"in_norm_w": ones,
                           "in_proj": [random_q4(r, HIDDEN, gen, device) for r in (8192, 4096, 32, 32)],
                           "out_proj": random_q4(HIDDEN, 4096, gen, device), "params": dn_params})
    return layers
