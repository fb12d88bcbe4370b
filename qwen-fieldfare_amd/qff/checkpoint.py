"""Weight and state wire format: an MLX safetensors checkpoint to the tensors
the entry points take, and the per-layer recurrent / KV state layout.

Reference: QwenQ4ActiveExpertStreamingRunner.swift:505-680 reads the
checkpoint (model.safetensors.index.json + shards, mmap'd; tensors located
by name through the shards' JSON headers) and :758-817 copies each layer's
quantized projections into a DenseLayerArena (Runner:6-59); per-layer
constants (conv1d weight, A_log, dt_bias, norms) are decoded from bf16 to
fp32 (:558-572, 636-640). Here the same names map to device tensors:

  DeltaNet layer l (l % 4 != 3), prefix language_model.model.layers.{l}.
    linear_attn.in_proj_{qkv,z,b,a}.{weight,scales,biases}  Q4 parts, the
        fused in-projection's order (qkv 8192, z 4096, b 32, a 32 rows)
    linear_attn.out_proj.*                                  Q4 [2048, 4096]
    linear_attn.conv1d.weight [8192, 4, 1] or [8192, 1, 4]  -> conv_w
        [8192, 4] fp32, c * 4 + j with tap 3 on the newest token
    linear_attn.A_log, dt_bias [32], norm.weight [128]      -> fp32
  full-attention layer (l % 4 == 3)
    self_attn.{q,k,v}_proj.*, o_proj.*                      Q4 parts
    self_attn.{q,k}_norm.weight [256]                       -> fp32
  every layer: input_layernorm.weight [2048] (used as is, deltanet.metal
    :18-53), mlp.gate.* (Q8 router [256, 2048]).

Quantized tensors stay in the checkpoint's bytes (uint32 words viewed as
int32, bf16 scales/biases), so no repacking happens on load: the kernels
read the MLX layout directly.

State (zero-copy with the reference's buffers, Runner:711-742): conv state
[B, 8192, 4] fp32 (slot 3 newest; the reference keeps [8192, 4] per
sequence), SSM state [B, 32, 128, 128] fp32 (row = v, column = k), K and V
caches [B, max_ctx, 2, 256] (token-major, bf16 where the reference uses
fp16). A snapshot is a copy of these tensors; restoring it and continuing
with qff.deltanet_prefill / qff.gqa_prefill (start_pos = the snapshot's
length) resumes an incremental prefill.

The reader parses the safetensors container itself (an 8-byte little-endian
header length, a JSON header, raw little-endian data) and never unpickles
anything.
"""
from __future__ import annotations

import json
import mmap
import os

import numpy as np
import torch

_DTYPES = {"U32": np.uint32, "I32": np.int32, "BF16": np.uint16, "F16": np.float16, "F32": np.float32,
           "U8": np.uint8}


class SafetensorsFile:
    """Read-only view of one .safetensors shard."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        n = int.from_bytes(self._mm[:8], "little")
        if n <= 0 or 8 + n > len(self._mm):
            raise ValueError(f"invalid safetensors header length in {path}")
        self.header = json.loads(self._mm[8:8 + n].decode("utf-8"))
        self._base = 8 + n

    def names(self):
        return [k for k in self.header if k != "__metadata__"]

    def raw(self, name: str):
        """(numpy array over the file's bytes, safetensors dtype string)."""
        meta = self.header[name]
        dt = meta["dtype"]
        if dt not in _DTYPES:
            raise ValueError(f"{name}: unsupported dtype {dt}")
        b0, b1 = meta["data_offsets"]
        arr = np.frombuffer(self._mm, dtype=_DTYPES[dt], count=(b1 - b0) // np.dtype(_DTYPES[dt]).itemsize,
                            offset=self._base + b0)
        return arr.reshape(meta["shape"]), dt

    def close(self):
        self._mm.close()
        self._f.close()


class Checkpoint:
    """A checkpoint directory: model.safetensors.index.json (weight_map) and
    its shards, or a single model.safetensors."""

    def __init__(self, directory: str, prefix: str = "language_model.model."):
        self.dir = directory
        self.prefix = prefix
        idx = os.path.join(directory, "model.safetensors.index.json")
        self._files = {}
        if os.path.exists(idx):
            with open(idx) as f:
                self.weight_map = json.load(f)["weight_map"]
        else:
            if not os.path.exists(os.path.join(directory, "model.safetensors")):
                raise FileNotFoundError(os.path.join(directory, "model.safetensors"))
            self.weight_map = {k: "model.safetensors" for k in self._file("model.safetensors").names()}

    def _file(self, shard: str) -> SafetensorsFile:
        if shard not in self._files:
            self._files[shard] = SafetensorsFile(os.path.join(self.dir, shard))
        return self._files[shard]

    def raw(self, name: str):
        if name not in self.weight_map:
            raise KeyError(name)
        return self._file(self.weight_map[name]).raw(name)

    def fp32(self, name: str, device="cuda") -> torch.Tensor:
        """A bf16 / f16 / f32 tensor decoded to fp32, as the reference's
        decodeBF16Tensor does."""
        a, dt = self.raw(name)
        if dt == "BF16":
            f = (a.astype(np.uint32) << 16).view(np.float32)
        else:
            f = a.astype(np.float32)
        return torch.from_numpy(np.ascontiguousarray(f)).to(device)

    def quant(self, stem: str, device="cuda"):
        """(weight int32 [rows, cols/8 or cols/4], scales, biases) of a
        quantized linear layer, bytes unchanged."""
        w, wdt = self.raw(stem + ".weight")
        if wdt not in ("U32", "I32"):
            raise ValueError(f"{stem}.weight: expected packed uint32, got {wdt}")
        wt = torch.from_numpy(np.array(w, copy=True).view(np.int32)).to(device)
        out = [wt]
        for part in ("scales", "biases"):
            a, dt = self.raw(f"{stem}.{part}")
            if dt == "BF16":
                t = torch.from_numpy(np.array(a, copy=True).view(np.int16)).view(torch.bfloat16)
            elif dt == "F16":
                t = torch.from_numpy(np.array(a, copy=True))
            else:
                raise ValueError(f"{stem}.{part}: expected bf16 or f16, got {dt}")
            out.append(t.to(device))
        return tuple(out)

    def close(self):
        for f in self._files.values():
            f.close()
        self._files.clear()

    # ---- per-layer views ---------------------------------------------------
    def layer_kind(self, l: int) -> str:
        return "gqa" if (self.prefix + f"layers.{l}.self_attn.q_proj.weight") in self.weight_map else "dn"

    def deltanet_layer(self, l: int, device="cuda") -> dict:
        p = self.prefix + f"layers.{l}."
        conv = self.fp32(p + "linear_attn.conv1d.weight", device).reshape(8192, 4).contiguous()
        return {
            "in_norm_w": self.fp32(p + "input_layernorm.weight", device),
            "in_proj": [self.quant(p + f"linear_attn.in_proj_{n}", device) for n in ("qkv", "z", "b", "a")],
            "out_proj": self.quant(p + "linear_attn.out_proj", device),
            "params": {
                "a_log": self.fp32(p + "linear_attn.A_log", device),
                "dt_bias": self.fp32(p + "linear_attn.dt_bias", device),
                "conv_w": conv,
                "norm_w": self.fp32(p + "linear_attn.norm.weight", device),
            },
            "router": self.quant(p + "mlp.gate", device) if (p + "mlp.gate.weight") in self.weight_map else None,
        }

    def gqa_layer(self, l: int, device="cuda") -> dict:
        p = self.prefix + f"layers.{l}."
        return {
            "in_norm_w": self.fp32(p + "input_layernorm.weight", device),
            "in_proj": [self.quant(p + f"self_attn.{n}_proj", device) for n in ("q", "k", "v")],
            "out_proj": self.quant(p + "self_attn.o_proj", device),
            "params": {
                "q_norm_w": self.fp32(p + "self_attn.q_norm.weight", device),
                "k_norm_w": self.fp32(p + "self_attn.k_norm.weight", device),
            },
            "router": self.quant(p + "mlp.gate", device) if (p + "mlp.gate.weight") in self.weight_map else None,
        }


# ---- state -----------------------------------------------------------------
def new_deltanet_state(batch: int, device="cuda") -> dict:
    """Zero conv state [B, 8192, 4] and SSM state [B, 32, 128, 128] (fp32)."""
    return {"conv_state": torch.zeros(batch, 8192, 4, device=device),
            "ssm_state": torch.zeros(batch, 32, 128, 128, device=device)}


def new_gqa_state(batch: int, max_ctx: int, device="cuda") -> dict:
    """Zero bf16 K and V caches [B, max_ctx, 2, 256]."""
    return {"k_cache": torch.zeros(batch, max_ctx, 2, 256, dtype=torch.bfloat16, device=device),
            "v_cache": torch.zeros(batch, max_ctx, 2, 256, dtype=torch.bfloat16, device=device)}


def snapshot(state: dict, length: int | None = None) -> dict:
    """A copy of a layer's state (KV caches only up to `length` positions
    when given)."""
    out = {}
    for k, v in state.items():
        if length is not None and k in ("k_cache", "v_cache"):
            out[k] = v[:, :length].clone()
        else:
            out[k] = v.clone()
    return out


def restore(state: dict, snap: dict) -> None:
    """Write a snapshot back into a layer's state tensors in place."""
    for k, v in snap.items():
        if k in ("k_cache", "v_cache") and v.shape[1] != state[k].shape[1]:
            state[k][:, :v.shape[1]].copy_(v)
        else:
            state[k].copy_(v)
