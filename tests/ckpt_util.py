"""A writer for small synthetic MLX-layout safetensors checkpoints (test
data only): the container is an 8-byte little-endian header length, a JSON
header {name: {dtype, shape, data_offsets}}, then the raw bytes."""
import json
import os

import numpy as np

from qff import synth


def write_safetensors(path, tensors):
    """tensors: name -> (numpy array, safetensors dtype string)."""
    header, blobs, off = {}, [], 0
    for name, (arr, dt) in tensors.items():
        b = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    hb = json.dumps(header).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    with open(path, "wb") as f:
        f.write(len(hb).to_bytes(8, "little"))
        f.write(hb)
        for b in blobs:
            f.write(b)


def _q4(tensors, stem, rows, cols, seed):
    w, s, b = synth.q4_weight(rows, cols, seed=seed, sb_dtype="bf16")
    tensors[stem + ".weight"] = (w, "U32")
    tensors[stem + ".scales"] = (s, "BF16")
    tensors[stem + ".biases"] = (b, "BF16")
    return w, s, b


def make_checkpoint(directory, conv_shape=(8192, 4, 1)):
    """Layer 0 Gated DeltaNet, layer 3 full attention, both with a Q8 router;
    two shards and an index. Returns the source arrays by tensor name."""
    os.makedirs(directory, exist_ok=True)
    rng = np.random.default_rng(7)
    pre = "language_model.model.layers."
    t0, t1 = {}, {}
    src = {}
    p = pre + "0."
    for n, rows in (("qkv", 8192), ("z", 4096), ("b", 32), ("a", 32)):
        src[n] = _q4(t0, p + f"linear_attn.in_proj_{n}", rows, 2048, seed=rows + 1)
    src["out"] = _q4(t0, p + "linear_attn.out_proj", 2048, 4096, seed=5)
    conv = synth._bf16_bits(rng.standard_normal((8192, 4)).astype(np.float32) * 0.5)
    src["conv"] = conv
    t0[p + "linear_attn.conv1d.weight"] = (conv.reshape(conv_shape), "BF16")
    for n, size in (("A_log", 32), ("dt_bias", 32), ("norm.weight", 128)):
        a = synth._bf16_bits(rng.standard_normal(size).astype(np.float32))
        src[n] = a
        t0[p + f"linear_attn.{n}"] = (a, "BF16")
    src["in_norm0"] = synth._bf16_bits(1 + 0.1 * rng.standard_normal(2048).astype(np.float32))
    t0[p + "input_layernorm.weight"] = (src["in_norm0"], "BF16")
    w, s, b = synth.q8_weight(256, 2048, seed=9)
    t0[p + "mlp.gate.weight"], t0[p + "mlp.gate.scales"], t0[p + "mlp.gate.biases"] = (w, "U32"), (s, "BF16"), (b, "BF16")
    src["router0"] = (w, s, b)
    p = pre + "3."
    for n, rows in (("q", 8192), ("k", 512), ("v", 512)):
        src[n] = _q4(t1, p + f"self_attn.{n}_proj", rows, 2048, seed=rows + 3)
    src["o"] = _q4(t1, p + "self_attn.o_proj", 2048, 4096, seed=11)
    for n in ("q_norm", "k_norm"):
        a = synth._bf16_bits(1 + 0.1 * rng.standard_normal(256).astype(np.float32))
        src[n] = a
        t1[p + f"self_attn.{n}.weight"] = (a, "BF16")
    src["in_norm3"] = synth._bf16_bits(1 + 0.1 * rng.standard_normal(2048).astype(np.float32))
    t1[p + "input_layernorm.weight"] = (src["in_norm3"], "BF16")
    write_safetensors(os.path.join(directory, "model-00001-of-00002.safetensors"), t0)
    write_safetensors(os.path.join(directory, "model-00002-of-00002.safetensors"), t1)
    wm = {k: "model-00001-of-00002.safetensors" for k in t0}
    wm.update({k: "model-00002-of-00002.safetensors" for k in t1})
    with open(os.path.join(directory, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)
    return src
