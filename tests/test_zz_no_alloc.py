"""qff_gqa_decode_static, the allocation-free variant of qff_gqa_decode
(split-KV partials in the library's fixed device array instead of a
context's workspace), against qff_gqa_decode through the C ABI: calls in a
row, each with a smaller batch and context than the last (batch 1 takes the
single-sequence split), each bit-identical with the context entry point
(same kernels; the context is sized so both split the positions the same
way), the caches included, on bf16 and on fp16 caches; oversized batches
are rejected before anything is launched."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import DEV, bf16_tensor, f16_tensor, f32_tensor
from oracle import oracle as O
from qff import synth

pytestmark = pytest.mark.gpu


def _call_static(prm, qg, kn, vn, kc, vc, pos, out, B, max_ctx):
    from qff._lib import lib
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return lib().qff_gqa_decode_static(st, ctypes.byref(prm), qg.data_ptr(), kn.data_ptr(), vn.data_ptr(), 1,
                                       kc.data_ptr(), vc.data_ptr(), pos.data_ptr(), out.data_ptr(),
                                       0, B, max_ctx)


@pytest.mark.parametrize("kv_f16", [0, 1])
def test_gqa_decode_static_matches_context_entry(hip, kv_f16):
    import qff
    from qff._lib import GqaParams
    p = {k: f32_tensor(v) for k, v in synth.gqa_params().items()}
    prm = GqaParams(p["q_norm_w"].data_ptr(), p["k_norm_w"].data_ptr(), 1e7, 64, 1.0 / 16, 1e-6, kv_f16)
    # 16 x 2 x 128 = 4096 partial slots: the static array's count, so both
    # entry points pick the same chunk length
    ctx = qff.Context(max_batch=16, max_ctx=8192, max_prefill_tokens=1)
    for B, max_ctx, seed in ((8, 8192, 1), (3, 2048, 2), (1, 1024, 3)):
        print(f"gqa_decode_static B={B} max_ctx={max_ctx} kv_f16={kv_f16}", flush=True)
        rng = np.random.default_rng(seed)
        inp = synth.gqa_decode_inputs(B, max_ctx, seed=seed, lengths=rng.integers(1, max_ctx + 1, B))
        qg, kn, vn = (bf16_tensor(inp[k]) for k in ("q_gate", "k_new", "v_new"))
        pos = torch.from_numpy(inp["positions"]).to(DEV)
        if kv_f16:
            kc_a = f16_tensor(O.f32_to_f16(O.bf16_to_f32(inp["k_cache"])))
            vc_a = f16_tensor(O.f32_to_f16(O.bf16_to_f32(inp["v_cache"])))
        else:
            kc_a, vc_a = bf16_tensor(inp["k_cache"]), bf16_tensor(inp["v_cache"])
        kc_b, vc_b = kc_a.clone(), vc_a.clone()
        ref = qff.gqa_decode(ctx, p, qg, kn, vn, kc_a, vc_a, pos, out_dtype=torch.float32)
        out = torch.full((B, 16, 256), float("nan"), device=DEV)
        assert _call_static(prm, qg, kn, vn, kc_b, vc_b, pos, out, B, max_ctx) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert torch.equal(kc_a.view(torch.int16), kc_b.view(torch.int16))
        assert torch.equal(vc_a.view(torch.int16), vc_b.view(torch.int16))
    ctx.close()


def test_gqa_decode_static_rejects_oversized_batch(hip):
    from qff._lib import GqaParams
    p = {k: f32_tensor(v) for k, v in synth.gqa_params().items()}
    prm = GqaParams(p["q_norm_w"].data_ptr(), p["k_norm_w"].data_ptr(), 1e7, 64, 1.0 / 16, 1e-6)
    B, max_ctx = 65, 16
    qg = torch.zeros(B, 16, 512, dtype=torch.bfloat16, device=DEV)
    kn = torch.zeros(B, 2, 256, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(B, max_ctx, 2, 256, dtype=torch.bfloat16, device=DEV)
    pos = torch.zeros(B, dtype=torch.int32, device=DEV)
    out = torch.zeros(B, 16, 256, device=DEV)
    assert _call_static(prm, qg, kn, kn, kc, kc.clone(), pos, out, B, max_ctx) == -4
    assert _call_static(prm, qg, kn, kn, kc, kc.clone(), pos, out, 0, max_ctx) == -1


def test_gqa_decode_static_graph_replay(hip):
    """The static entry point captured in a HIP graph (after one eager call,
    which resolves the array's address) and replayed three times, with eager
    work and synchronisations between the replays: every replay equals the
    context entry point's result bit for bit, and the appended cache rows too."""
    import qff
    from qff._lib import GqaParams
    p = {k: f32_tensor(v) for k, v in synth.gqa_params().items()}
    prm = GqaParams(p["q_norm_w"].data_ptr(), p["k_norm_w"].data_ptr(), 1e7, 64, 1.0 / 16, 1e-6)
    B, max_ctx = 4, 4096
    print(f"gqa_decode_static graph replay B={B} max_ctx={max_ctx}", flush=True)
    # 32 x 2 x 64 = 4096 slots: the same chunk cap as the static array
    ctx = qff.Context(max_batch=32, max_ctx=max_ctx, max_prefill_tokens=1)
    inp = synth.gqa_decode_inputs(B, max_ctx, seed=31, lengths=[4096, 1, 777, 3000])
    qg, kn, vn = (bf16_tensor(inp[k]) for k in ("q_gate", "k_new", "v_new"))
    pos = torch.from_numpy(inp["positions"]).to(DEV)
    kc_a, vc_a = bf16_tensor(inp["k_cache"]), bf16_tensor(inp["v_cache"])
    kc_b, vc_b = kc_a.clone(), vc_a.clone()
    ref = qff.gqa_decode(ctx, p, qg, kn, vn, kc_a, vc_a, pos, out_dtype=torch.float32)
    out = torch.full((B, 16, 256), float("nan"), device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        assert _call_static(prm, qg, kn, vn, kc_b, vc_b, pos, out, B, max_ctx) == 0   # eager, sets up
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        assert _call_static(prm, qg, kn, vn, kc_b, vc_b, pos, out, B, max_ctx) == 0
    for r in range(3):
        out.fill_(float("nan"))
        junk = torch.randn(1 << 20, device=DEV).sum()   # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        assert torch.equal(out, ref), f"replay {r}"
        assert torch.equal(kc_a.view(torch.int16), kc_b.view(torch.int16))
        assert torch.equal(vc_a.view(torch.int16), vc_b.view(torch.int16))
    ctx.close()
