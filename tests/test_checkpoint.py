"""The checkpoint / state wire format on the CPU: tensors found by name
across shards, quantized bytes unchanged, bf16 constants decoded to fp32,
the conv1d weight in c * 4 + j order from either MLX or PyTorch shape, and
state snapshots that restore in place. The tensor names are those the
reference reads (QwenQ4ActiveExpertStreamingRunner.swift:537-680)."""
import numpy as np
import pytest
import torch

from ckpt_util import make_checkpoint
from oracle import oracle as O
from qff import checkpoint as C


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    src = make_checkpoint(str(d))
    return C.Checkpoint(str(d)), src


def test_layer_kinds_and_quantized_bytes(ckpt):
    ck, src = ckpt
    assert ck.layer_kind(0) == "dn" and ck.layer_kind(3) == "gqa"
    dn = ck.deltanet_layer(0, device="cpu")
    for (w, s, b), n in zip(dn["in_proj"], ("qkv", "z", "b", "a")):
        sw, ss, sb = src[n]
        assert np.array_equal(w.numpy().view(np.uint32), sw)
        assert s.dtype == torch.bfloat16 and np.array_equal(s.view(torch.int16).numpy().view(np.uint16), ss)
        assert np.array_equal(b.view(torch.int16).numpy().view(np.uint16), sb)
    w, s, b = dn["out_proj"]
    assert w.shape == (2048, 512)
    rw, rs, rb = dn["router"]
    assert np.array_equal(rw.numpy().view(np.uint32), src["router0"][0])
    gq = ck.gqa_layer(3, device="cpu")
    assert [t[0].shape[0] for t in gq["in_proj"]] == [8192, 512, 512]


def test_constants_decode_to_fp32(ckpt):
    ck, src = ckpt
    dn = ck.deltanet_layer(0, device="cpu")
    assert np.array_equal(dn["params"]["conv_w"].numpy(), O.bf16_to_f32(src["conv"]))
    assert np.array_equal(dn["params"]["a_log"].numpy(), O.bf16_to_f32(src["A_log"]))
    assert np.array_equal(dn["params"]["norm_w"].numpy(), O.bf16_to_f32(src["norm.weight"]))
    assert np.array_equal(dn["in_norm_w"].numpy(), O.bf16_to_f32(src["in_norm0"]))
    gq = ck.gqa_layer(3, device="cpu")
    assert np.array_equal(gq["params"]["q_norm_w"].numpy(), O.bf16_to_f32(src["q_norm"]))


def test_conv_weight_layout_from_either_shape(tmp_path):
    src = make_checkpoint(str(tmp_path), conv_shape=(8192, 1, 4))
    ck = C.Checkpoint(str(tmp_path))
    conv = ck.deltanet_layer(0, device="cpu")["params"]["conv_w"]
    assert conv.shape == (8192, 4)
    assert np.array_equal(conv.numpy(), O.bf16_to_f32(src["conv"]))   # c * 4 + j, tap 3 newest


def test_missing_tensor_and_bad_header(tmp_path):
    make_checkpoint(str(tmp_path))
    ck = C.Checkpoint(str(tmp_path))
    with pytest.raises(KeyError):
        ck.raw("language_model.model.layers.1.linear_attn.A_log")
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes((10 ** 9).to_bytes(8, "little") + b"{}")
    with pytest.raises(ValueError):
        C.SafetensorsFile(str(bad))


def test_state_snapshot_restore():
    st = C.new_deltanet_state(2, device="cpu")
    st["ssm_state"].normal_()
    snap = C.snapshot(st)
    saved = st["ssm_state"].clone()
    st["ssm_state"].zero_()
    C.restore(st, snap)
    assert torch.equal(st["ssm_state"], saved)
    kv = C.new_gqa_state(1, 64, device="cpu")
    kv["k_cache"][:, :10] = 1.0
    part = C.snapshot(kv, length=10)
    assert part["k_cache"].shape == (1, 10, 2, 256)
    kv["k_cache"].zero_()
    C.restore(kv, part)
    assert torch.all(kv["k_cache"][:, :10] == 1.0) and torch.all(kv["k_cache"][:, 10:] == 0)
