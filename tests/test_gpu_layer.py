"""A decoder layer's attention block assembled from the entry points on
weights read through the checkpoint wire format: input RMSNorm fused into
the in-projections (qff_q4_norm_matmul_parts), the layer core, and the
out-projection adding into the residual stream in place -- the encoder
sequence of QwenQ4ActiveExpertStreamingRunner.swift:972-1040 -- against the
oracle run in the same order (rmsnorm, Q4 matvecs in the reference's
factored order, the sequential DeltaNet step, Q4 out-projection, residual
add). The products take the normed activations as bf16(x w_norm) scaled by
the inverse RMS afterwards, and the out-projection takes the layer core's
output as bf16; with the oracle fed the same roundings the
layer output must agree to 1e-3 of its largest value and the updated state
to rel 1e-3, and against the unrounded reference order to 1e-2 / 5e-2
(the state of one step carries the bf16 rounding of k and v). A
wrong tensor mapping (a swapped part, a transposed conv weight, a missing
norm) is off by O(1)."""
import numpy as np
import pytest
import torch

from ckpt_util import make_checkpoint
from gpu_util import DEV, state_rel_err
from oracle import oracle as O
from qff import checkpoint as C

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt_gpu")
    src = make_checkpoint(str(d))
    return C.Checkpoint(str(d)), src


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("batch", [1, 3])
def test_deltanet_layer_decode_from_checkpoint(hip, ckpt, batch):
    import qff
    print(f"deltanet layer from checkpoint batch={batch}", flush=True)
    ck, _ = ckpt
    L = ck.deltanet_layer(0, device=DEV)
    rng = np.random.default_rng(batch)
    h0 = rng.standard_normal((batch, 2048)).astype(np.float32)
    conv0 = np.zeros((batch, 8192, 4), np.float32)
    conv0[:, :, 1:] = rng.standard_normal((batch, 8192, 3)).astype(np.float32)
    ssm0 = (rng.standard_normal((batch, 32, 128, 128)) * 0.02).astype(np.float32)
    ctx = qff.Context(max_batch=32, max_ctx=64, max_prefill_tokens=64)
    h = torch.from_numpy(h0).to(DEV)
    conv = torch.from_numpy(conv0).to(DEV)
    ssm = torch.from_numpy(ssm0).to(DEV)
    qkv, z, bb, aa = qff.q4_norm_matmul_parts(ctx, L["in_proj"], h, L["in_norm_w"], 1e-6)
    core = qff.deltanet_decode(ctx, L["params"], qkv, z, aa, bb, conv, ssm, out_dtype=torch.float32)
    qff.q4_matmul_parts(ctx, [L["out_proj"]], core, outs=(h,), residuals=(h,))
    torch.cuda.synchronize()

    prm = {k: _np(v) for k, v in L["params"].items()}
    in_w = _np(L["in_norm_w"])
    q4 = [tuple(t.cpu() for t in part) for part in L["in_proj"]]
    wo = tuple(t.cpu() for t in L["out_proj"])

    def mv(part, x):
        w, s, b = part
        return O.q4_matvec(w.numpy().view(np.uint32), s.view(torch.int16).numpy().view(np.uint16),
                           b.view(torch.int16).numpy().view(np.uint16), x, O.BF16)

    def layer(xn, m, round_core):
        r_qkv, r_z, r_b, r_a = (mv(p, xn) for p in q4)
        out, cs, ss = O.deltanet_sequence(r_qkv, r_z, r_a, r_b, prm["a_log"], prm["dt_bias"], prm["conv_w"],
                                          prm["norm_w"], conv0[m], ssm0[m])
        core = O.round_bf16(out[0]) if round_core else out[0]
        return h0[m] + mv(wo, core), ss

    for m in range(batch):
        got = _np(h)[m]
        # the products' own rounding of the normed activations
        inv = 1.0 / np.sqrt(np.mean(h0[m].astype(np.float64) ** 2) + 1e-6)
        xq = (O.round_bf16((h0[m] * in_w).astype(np.float32)).astype(np.float64) * inv).astype(np.float32)
        ref, ss = layer(xq, m, True)
        assert np.max(np.abs(got - ref)) <= 1e-3 * np.max(np.abs(ref))
        assert state_rel_err(_np(ssm)[m], ss) <= 1e-3
        # the reference order, fp32 throughout
        ref, ss = layer(O.rmsnorm(h0[m], in_w, 1e-6), m, False)
        assert np.max(np.abs(got - ref)) <= 1e-2 * np.max(np.abs(ref))
        assert state_rel_err(_np(ssm)[m], ss) <= 5e-2
        assert np.array_equal(_np(conv)[m][:, 1:3], conv0[m][:, 2:4])   # history shifted by one


def test_gqa_layer_projections_from_checkpoint(hip, ckpt):
    import qff
    ck, _ = ckpt
    L = ck.gqa_layer(3, device=DEV)
    x0 = np.random.default_rng(5).standard_normal((2, 2048)).astype(np.float32)
    ctx = qff.Context(max_batch=32, max_ctx=64, max_prefill_tokens=64)
    outs = qff.q4_norm_matmul_parts(ctx, L["in_proj"], torch.from_numpy(x0).to(DEV), L["in_norm_w"], 1e-6)
    torch.cuda.synchronize()
    in_w = _np(L["in_norm_w"])
    for part, o, rows in zip(L["in_proj"], outs, (8192, 512, 512)):
        w, s, b = (t.cpu() for t in part)
        assert o.shape == (2, rows)
        for m in range(2):
            ref = O.q4_matvec(w.numpy().view(np.uint32), s.view(torch.int16).numpy().view(np.uint16),
                              b.view(torch.int16).numpy().view(np.uint16), O.rmsnorm(x0[m], in_w, 1e-6), O.BF16)
            assert np.max(np.abs(_np(o)[m] - ref)) <= 1e-2 * np.max(np.abs(ref))
