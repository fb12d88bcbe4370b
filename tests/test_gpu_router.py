"""GPU parity of the MoE-router entry points (deltanet.metal:863-900,
2229-2329). qff_q8_dequant must be bit-exact with the closed form.
qff_router_top8: logits within rel 1e-5 (max-abs over max |logit|) of the
fp64 dense product; indices equal to the oracle's top-8 rule applied to the
kernel's own logits, and to the oracle's logits where the eight winners are
separated from the rest by more than the logit tolerance; scores within
1e-6 of the oracle's on the kernel's logits."""
import numpy as np
import pytest
import torch

from gpu_util import DEV, bf16_tensor, f16_tensor, f32_tensor, to_np
from oracle import oracle as O
from qff import synth

pytestmark = pytest.mark.gpu


def _w_gpu(w, s, b, sb):
    conv = f16_tensor if sb == "f16" else bf16_tensor
    return torch.from_numpy(w.view(np.int32)).to(DEV), conv(s), conv(b)


@pytest.mark.parametrize("rows,cols,sb", [(256, 2048, "bf16"), (17, 64, "f16"), (40, 4096, "bf16")])
def test_q8_dequant_bit_exact(hip, rows, cols, sb):
    import qff
    print(f"q8_dequant {rows}x{cols} {sb}", flush=True)
    w, s, b = synth.q8_weight(rows, cols, seed=rows + cols, sb_dtype=sb)
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    out = qff.q8_dequant(ctx, *_w_gpu(w, s, b, sb))
    torch.cuda.synchronize()
    ref = O.q8_dequant(w, s, b, O.F16 if sb == "f16" else O.BF16)
    assert np.array_equal(to_np(out).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("batch,experts,cols,xdt", [(1, 256, 2048, "f32"), (5, 256, 2048, "bf16"),
                                                    (32, 256, 2048, "f32"), (300, 256, 2048, "f32"),
                                                    (3, 64, 1024, "f32"), (2, 8, 4096, "bf16"),
                                                    (9, 100, 192, "f32")])
def test_router_top8(hip, batch, experts, cols, xdt):
    import qff
    print(f"router_top8 batch={batch} experts={experts} cols={cols} x={xdt}", flush=True)
    w, s, b = synth.q8_weight(experts, cols, seed=experts + cols + batch)
    rng = np.random.default_rng(batch)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    if xdt == "bf16":
        x = O.round_bf16(x)
        xt = bf16_tensor(O.f32_to_bf16(x))
    else:
        xt = f32_tensor(x)
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    idx, sc, lg = qff.router_top8(ctx, *_w_gpu(w, s, b, "bf16"), xt)
    torch.cuda.synchronize()
    idx, sc, lg = idx.cpu().numpy(), sc.cpu().numpy(), lg.cpu().numpy()
    dense = O.q8_dequant(w, s, b, O.BF16).astype(np.float64)
    ref_lg = x.astype(np.float64) @ dense.T
    tol = 1e-5 * np.max(np.abs(ref_lg))
    assert np.max(np.abs(lg - ref_lg)) <= tol
    for m in range(batch):
        oi, os_ = O.router_top8(lg[m])
        assert np.array_equal(idx[m], oi)
        assert np.allclose(sc[m], os_, atol=1e-6)
        # against the oracle's own logits where the ranking is unambiguous
        ol = O.router_logits(w, s, b, x[m], O.BF16)
        srt = np.sort(ol.astype(np.float64))[::-1]
        gaps = np.diff(srt[:9])
        if np.all(np.abs(gaps) > 4 * tol):
            assert np.array_equal(idx[m], O.router_top8(ol)[0])


def test_router_rejects_bad_calls(hip):
    import qff
    from qff._lib import lib
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    w, s, b = _w_gpu(*synth.q8_weight(300, 128, seed=1), "bf16")
    x = torch.zeros(1, 128, device=DEV)
    with pytest.raises(qff.QffError) as e:
        qff.router_top8(ctx, w, s, b, x)           # 300 experts > 256
    assert e.value.status == -2
    L = lib()
    assert L.qff_router_top8(ctx.handle, None, w.data_ptr(), s.data_ptr(), b.data_ptr(), 1, x.data_ptr(), 0,
                             None, None, None, 256, 128, 1) == -1
