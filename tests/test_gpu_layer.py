"""A decoder layer's attention block assembled from the entry points on
weights read through the checkpoint wire format: input RMSNorm fused into
the in-projections (qff_q4_norm_matmul_parts), the layer core, and the
out-projection adding into the residual stream in place -- the encoder
sequence of QwenQ4ActiveExpertStreamingRunner.swift:972-1040 (DeltaNet) and
:1041-1167 (full attention) -- against the oracle run in the same order
(rmsnorm, Q4 matvecs in the reference's factored fp32 order, the layer core,
Q4 out-projection, residual add; tests/layer_oracle.py).

Everything stays fp32 between the steps, as in the reference; the decode Q4
products take fp32 activations as bf16 hi + lo pairs, so a DeltaNet block
must match the reference order to 1e-4 of its largest residual update and
its state to rel 1e-4. A full-attention block differs by the reference's
own fp16 roundings of q and of the attention output (the cores round
differently), so its update must match to 5e-3 of its largest entry. A
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

    def layer(xn, m):
        r_qkv, r_z, r_b, r_a = (mv(p, xn) for p in q4)
        out, cs, ss = O.deltanet_sequence(r_qkv, r_z, r_a, r_b, prm["a_log"], prm["dt_bias"], prm["conv_w"],
                                          prm["norm_w"], conv0[m], ssm0[m])
        return h0[m] + mv(wo, out[0]), ss

    for m in range(batch):
        got = _np(h)[m]
        ref, ss = layer(O.rmsnorm(h0[m], in_w, 1e-6), m)
        e_upd = np.max(np.abs(got - ref)) / np.max(np.abs(ref - h0[m]))
        e_st = state_rel_err(_np(ssm)[m], ss)
        print(f"  seq {m}: update {e_upd:.3g}, state {e_st:.3g}", flush=True)
        assert e_upd <= 1e-4 and e_st <= 1e-4
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


@pytest.mark.parametrize("batch", [1, 3])
def test_gqa_layer_decode_from_checkpoint(hip, ckpt, batch):
    """A full-attention block from the checkpoint's layer-3 tensors through
    qff.stack (input RMSNorm + q|gate/k/v projections, qff_gqa_decode on the
    fp32 projections, o_proj added into the fp32 residual stream) against
    the oracle composed in the order of QwenQ4ActiveExpertStreamingRunner
    .swift:1041-1167: the residual update within 5e-3 of its largest entry;
    the caches change only at each sequence's position."""
    import qff
    import layer_oracle as LO
    from qff import stack as S
    print(f"gqa layer from checkpoint batch={batch}", flush=True)
    ck, _ = ckpt
    L = ck.gqa_layer(3, device=DEV)
    max_ctx = 64
    rng = np.random.default_rng(30 + batch)
    ctx = qff.Context(max_batch=4, max_ctx=max_ctx, max_prefill_tokens=64)
    st = S.AttentionStack(ctx, [L], batch, max_ctx, kinds=["gqa"])
    kc0 = O.f32_to_bf16(rng.standard_normal((batch, max_ctx, 2, 256)).astype(np.float32))
    vc0 = O.f32_to_bf16(rng.standard_normal((batch, max_ctx, 2, 256)).astype(np.float32))
    st.states[0]["k_cache"].copy_(torch.from_numpy(kc0.view(np.int16)).view(torch.bfloat16))
    st.states[0]["v_cache"].copy_(torch.from_numpy(vc0.view(np.int16)).view(torch.bfloat16))
    positions = np.array([5, 63, 0][:batch], np.int32)
    x0 = rng.standard_normal((batch, 2048)).astype(np.float32)
    x = torch.from_numpy(x0).to(DEV)
    st.decode_step(x, torch.from_numpy(positions).to(DEV))
    torch.cuda.synchronize()
    Lnp = LO.layer_to_np(L)
    got = _np(x)
    kg = st.states[0]["k_cache"].cpu().view(torch.int16).numpy().view(np.uint16)
    for m in range(batch):
        p = int(positions[m])
        ref = LO.gqa_layer(Lnp, x0[m], kc0[m].copy(), vc0[m].copy(), p)
        upd = got[m] - x0[m]
        e_r = np.max(np.abs(upd - (ref - x0[m]))) / np.max(np.abs(ref - x0[m]))
        print(f"  seq {m}: update vs reference order {e_r:.3g}", flush=True)
        assert e_r <= 5e-3
        mask = np.ones(max_ctx, bool)
        mask[p] = False
        assert np.array_equal(kg[m][mask], kc0[m][mask])
    ctx.close()
