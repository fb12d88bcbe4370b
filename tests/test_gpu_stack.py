"""The attention stack (qff.stack.AttentionStack: the per-layer schedule of
QwenQ4ActiveExpertStreamingRunner.swift:924-1167 with l % 4 == 3 full
attention, Runner:554-556) checked layer by layer against the oracle in the
reference's encoder order (tests/layer_oracle.py).

For every layer the oracle starts from the GPU's own layer input x (and the
layer's state before the step), so the comparison isolates that layer. The
stream and every intermediate are fp32 and the decode Q4 products take fp32
activations as bf16 hi + lo pairs, so
  * a DeltaNet layer's residual update must match the reference order to
    1e-4 of its largest entry, and its state to rel 1e-4;
  * a full-attention layer's update to 5e-3 of its largest entry (the
    reference rounds q and the attention output to fp16, the kernels keep
    more bits);
  * the conv history shifts bit-exactly (its new slot, the token's own
    projection, within 1e-5) and the KV caches change only at the new
    position.
The bench's config-4 step is this same object (bench.py bench_c4)."""
import numpy as np
import pytest
import torch

import layer_oracle as LO
from gpu_util import DEV, state_rel_err, to_np
from oracle import oracle as O
from qff import synth

pytestmark = pytest.mark.gpu


def _rel_max(got, ref):
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _make_stack(n_layers, B, max_ctx, seed):
    import qff
    from qff import stack as S
    g = torch.Generator(device=DEV).manual_seed(seed)
    dnp = {k: torch.from_numpy(v).to(DEV) for k, v in synth.deltanet_params().items()}
    gqp = {k: torch.from_numpy(v).to(DEV) for k, v in synth.gqa_params().items()}
    layers = S.random_layers(n_layers, g, dnp, gqp, device=DEV)
    # input-RMSNorm weights other than 1, so a missing norm weight shows
    for l, L in enumerate(layers):
        L["in_norm_w"] = 1.0 + 0.1 * torch.randn(2048, device=DEV, generator=g)
    ctx = qff.Context(max_batch=max(B, 1), max_ctx=max_ctx, max_prefill_tokens=64)
    st = S.AttentionStack(ctx, layers, B, max_ctx)
    for kind, s in zip(st.kinds, st.states):
        if kind == "dn":
            s["conv_state"].normal_(generator=g)
            s["ssm_state"].normal_(generator=g).mul_(0.02)
        else:
            s["k_cache"].copy_(torch.randn(s["k_cache"].shape, device=DEV, generator=g).to(torch.bfloat16))
            s["v_cache"].copy_(torch.randn(s["v_cache"].shape, device=DEV, generator=g).to(torch.bfloat16))
    return ctx, st


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def _check_step(st, x, positions, seqs, tol_dn=1e-4, tol_gqa=5e-3):
    """One decode step through every layer of `st`, each layer checked for
    the sequences in `seqs`."""
    pos_t = torch.from_numpy(np.asarray(positions, np.int32)).to(DEV)
    worst = {"dn": [0.0, 0.0], "gqa": [0.0]}
    for l in range(len(st.layers)):
        Lnp = LO.layer_to_np(st.layers[l])
        x_in = to_np(x).copy()
        S = st.states[l]
        if st.kinds[l] == "dn":
            conv0, ssm0 = to_np(S["conv_state"]).copy(), to_np(S["ssm_state"]).copy()
        else:
            kc0, vc0 = _bits(S["k_cache"]).copy(), _bits(S["v_cache"]).copy()
        st.layer_step(l, x, pos_t)
        torch.cuda.synchronize()
        x_out = to_np(x)
        for m in seqs:
            upd = x_out[m] - x_in[m]
            if st.kinds[l] == "dn":
                ref, cs, ss = LO.deltanet_layer(Lnp, x_in[m], conv0[m], ssm0[m])
                e = [_rel_max(upd, ref - x_in[m]), state_rel_err(to_np(S["ssm_state"])[m], ss)]
                cg = to_np(S["conv_state"])[m]
                # the history shifts bit-exactly; the new slot holds each side's
                # own fp32 projection of the token
                assert np.array_equal(cg[:, :3], cs[:, :3]), f"layer {l} seq {m}: conv history"
                assert np.max(np.abs(cg[:, 3] - cs[:, 3])) <= 1e-5 * np.max(np.abs(cs[:, 3]))
                worst["dn"] = [max(a, b) for a, b in zip(worst["dn"], e)]
                assert e[0] <= tol_dn and e[1] <= 1e-4, f"layer {l} seq {m}: {e}"
            else:
                p = int(positions[m])
                kr, vr = kc0[m].copy(), vc0[m].copy()
                ref = LO.gqa_layer(Lnp, x_in[m], kr, vr, p)
                e = [_rel_max(upd, ref - x_in[m])]
                worst["gqa"] = [max(a, b) for a, b in zip(worst["gqa"], e)]
                assert e[0] <= tol_gqa, f"layer {l} seq {m}: {e}"
                kg, vg = _bits(S["k_cache"])[m], _bits(S["v_cache"])[m]
                mask = np.ones(st.max_ctx, bool)
                mask[p] = False
                assert np.array_equal(kg[mask], kc0[m][mask]) and np.array_equal(vg[mask], vc0[m][mask])
                kk = O.bf16_to_f32(kr[p])
                assert np.all(np.abs(O.bf16_to_f32(kg[p]) - kk) <= np.maximum(2.0 ** -7 * np.abs(kk), 2.0 ** -16))
        print(f"  layer {l} ({st.kinds[l]}) ok", flush=True)
    print(f"worst errors: {worst}", flush=True)


@pytest.mark.parametrize("B", [1, 16])
def test_stack_two_steps_short_context(hip, B):
    """Eight layers (two groups of 3 DeltaNet + 1 full attention), two decode
    steps in a row (positions advance, states carry over), at context 256."""
    print(f"stack 8 layers B={B}", flush=True)
    max_ctx = 256
    ctx, st = _make_stack(8, B, max_ctx, seed=100 + B)
    rng = np.random.default_rng(B)
    positions = rng.integers(0, max_ctx - 2, B)
    g = torch.Generator(device=DEV).manual_seed(B)
    x = torch.randn(B, 2048, device=DEV, generator=g)
    seqs = range(B) if B <= 4 else [0, 7, B - 1]
    for step in range(2):
        print(f" step {step} positions {positions[:4]}", flush=True)
        _check_step(st, x, positions + step, seqs)
    ctx.close()


def test_stack_config4_shape_one_group(hip):
    """The bench's config-4 shapes for one group of four layers: batch 16 at
    32K context (every sequence at position 32767, as bench.py times it),
    every sequence checked."""
    B, L = 16, 32768
    print(f"stack config-4 shape B={B} L={L}", flush=True)
    ctx, st = _make_stack(4, B, L, seed=44)
    g = torch.Generator(device=DEV).manual_seed(4)
    x = torch.randn(B, 2048, device=DEV, generator=g)
    _check_step(st, x, np.full(B, L - 1), seqs=range(B))
    ctx.close()


def test_stack_config4_single_sequence_64k(hip):
    """Config 4's single-sequence step: one group of four layers at batch 1
    and 64K context (position 65535, as bench.py times it), two steps in a
    row (positions 65534 and 65535, the cache's last two), the second on
    the states and cache the first left."""
    B, L = 1, 65536
    print(f"stack config-4 shape B={B} L={L}", flush=True)
    ctx, st = _make_stack(4, B, L, seed=64)
    g = torch.Generator(device=DEV).manual_seed(64)
    x = torch.randn(B, 2048, device=DEV, generator=g)
    for step, pos in enumerate((L - 2, L - 1)):
        print(f" step {step} position {pos}", flush=True)
        _check_step(st, x, np.full(B, pos), seqs=[0])
    ctx.close()
