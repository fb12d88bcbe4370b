"""GPU parity of the affine-Q4 entry points.

qff_q4_dequant must be bit-exact with the closed form
(QwenQ4ActiveExpertStreamingRunner.swift:899-922) for f16 and bf16 scales.
qff_q4_matmul is checked against an fp64 product of the dequantized matrix:
with bf16 activations (exact MFMA operands) the relative Frobenius error must
stay <= 1e-5 (fp32 accumulation order only); with fp32 activations, which the
matrix cores take rounded to bf16, <= 1e-2 against the reference's own fp32
factored order (deltanet.metal:816-861)."""
import numpy as np
import pytest
import torch

from gpu_util import DEV, bf16_tensor, f16_tensor, f32_tensor, to_np
from oracle import oracle as O
from qff import synth

pytestmark = pytest.mark.gpu


def _w_gpu(w, s, b, sb):
    wt = torch.from_numpy(w.view(np.int32)).to(DEV)
    conv = f16_tensor if sb == "f16" else bf16_tensor
    return wt, conv(s), conv(b)


@pytest.mark.parametrize("rows,cols,sb", [(512, 2048, "f16"), (2048, 4096, "bf16"), (17, 64, "f16"),
                                          (8192, 2048, "bf16")])
def test_q4_dequant_bit_exact(hip, rows, cols, sb):
    import qff
    print(f"q4_dequant {rows}x{cols} {sb}", flush=True)
    w, s, b = synth.q4_weight(rows, cols, seed=rows + cols, sb_dtype=sb)
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    out = qff.q4_dequant(ctx, *_w_gpu(w, s, b, sb))
    torch.cuda.synchronize()
    ref = O.q4_dequant(w, s, b, O.F16 if sb == "f16" else O.BF16)
    assert np.array_equal(to_np(out).view(np.uint32), ref.view(np.uint32))


def _rel(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("rows,cols,batch", [(8192, 2048, 1), (512, 2048, 5), (4096, 2048, 16),
                                             (2048, 4096, 32), (100, 2048, 33), (32, 2048, 1),
                                             # 64-row workgroups (batch >= 2, >= 8192 rows), ragged end
                                             (8192, 2048, 2), (8200, 2048, 17), (9216, 2048, 32),
                                             # many-token GEMM path (batch >= 64), ragged tiles included
                                             (512, 2048, 64), (100, 2048, 300), (8192, 2048, 256),
                                             (2048, 4096, 130), (512, 2048, 8192)])
def test_q4_matmul_bf16_activations(hip, rows, cols, batch):
    import qff
    print(f"q4_matmul {rows}x{cols} batch={batch}", flush=True)
    w, s, b = synth.q4_weight(rows, cols, seed=rows * 3 + batch)
    rng = np.random.default_rng(batch)
    xb = O.f32_to_bf16(rng.standard_normal((batch, cols)).astype(np.float32))
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    y = qff.q4_matmul(ctx, *_w_gpu(w, s, b, "f16"), bf16_tensor(xb))
    torch.cuda.synchronize()
    dense = O.q4_dequant(w, s, b, O.F16).astype(np.float64)
    ref = O.bf16_to_f32(xb).astype(np.float64) @ dense.T
    assert _rel(to_np(y), ref) <= 1e-5


def test_q4_matmul_f32_activations_vs_reference_order(hip):
    import qff
    rows, cols = 2048, 4096
    w, s, b = synth.q4_weight(rows, cols, seed=99)
    x = np.random.default_rng(5).standard_normal((2, cols)).astype(np.float32)
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    y = qff.q4_matmul(ctx, *_w_gpu(w, s, b, "f16"), f32_tensor(x))
    yb = qff.q4_matmul(ctx, *_w_gpu(w, s, b, "f16"), f32_tensor(x), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    for m in range(2):
        ref = O.q4_matvec(w, s, b, x[m])
        assert _rel(to_np(y)[m], ref) <= 1e-2
        assert _rel(to_np(yb)[m], ref) <= 1e-2


def test_q4_gemv_f32_activations_64_row_workgroups(hip):
    """Decode batch over >= 8192 rows (four row tiles per workgroup) with fp32
    activations: the product matches the fp64 product with bf16-rounded x."""
    import qff
    rows, cols, batch = 8256, 2048, 9
    w, s, b = synth.q4_weight(rows, cols, seed=8)
    x = np.random.default_rng(9).standard_normal((batch, cols)).astype(np.float32)
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    y = qff.q4_matmul(ctx, *_w_gpu(w, s, b, "bf16"), f32_tensor(x))
    torch.cuda.synchronize()
    dense = O.q4_dequant(w, s, b, O.BF16).astype(np.float64)
    ref = O.round_bf16(x).astype(np.float64) @ dense.T
    assert _rel(to_np(y), ref) <= 1e-5


def test_q4_gemm_f32_activations_round_like_bf16(hip):
    """Many-token path with fp32 activations: the matrix cores take x rounded
    to bf16, so the product matches the fp64 product with bf16-rounded x."""
    import qff
    rows, cols, batch = 640, 2048, 96
    w, s, b = synth.q4_weight(rows, cols, seed=7)
    x = np.random.default_rng(6).standard_normal((batch, cols)).astype(np.float32)
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    y = qff.q4_matmul(ctx, *_w_gpu(w, s, b, "f16"), f32_tensor(x))
    torch.cuda.synchronize()
    dense = O.q4_dequant(w, s, b, O.F16).astype(np.float64)
    ref = O.round_bf16(x).astype(np.float64) @ dense.T
    assert _rel(to_np(y), ref) <= 1e-5


def test_q4_rejects_bad_shapes(hip):
    import qff
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    w = torch.zeros(4, 12, dtype=torch.int32, device=DEV)          # cols = 96: not a multiple of 64
    s = torch.zeros(4, 1, dtype=torch.float16, device=DEV)
    with pytest.raises(qff.QffError) as e:
        qff.q4_dequant(ctx, w, s, s)
    assert e.value.status == -2


@pytest.mark.parametrize("batch", [1, 3, 16, 32, 40])
def test_q4_matmul_parts_match_single_products(hip, batch):
    """The four-part DeltaNet in-projection shape (qkv 8192, z 4096, b 32,
    a 32 rows; bf16, bf16, f32, f32 outputs) in one call: each part equals
    the single-matrix product bit for bit (same kernel per row block), and
    the first part matches the fp64 dequantized product."""
    import qff
    print(f"q4_matmul_parts batch={batch}", flush=True)
    cols = 2048
    shapes = [(8192, torch.bfloat16), (4096, torch.bfloat16), (32, torch.float32), (32, torch.float32)]
    ws = [synth.q4_weight(r, cols, seed=11 * r + batch) for r, _ in shapes]
    rng = np.random.default_rng(100 + batch)
    xb = O.f32_to_bf16(rng.standard_normal((batch, cols)).astype(np.float32))
    ctx = qff.Context(max_batch=32, max_ctx=64, max_prefill_tokens=64)
    parts = [_w_gpu(w, s, b, "f16") for w, s, b in ws]
    x = bf16_tensor(xb)
    outs = qff.q4_matmul_parts(ctx, parts, x, out_dtypes=[dt for _, dt in shapes])
    singles = [qff.q4_matmul(ctx, *pp, x, out_dtype=dt) for pp, (_, dt) in zip(parts, shapes)]
    torch.cuda.synchronize()
    for o, s1 in zip(outs, singles):
        assert o.dtype == s1.dtype and torch.equal(o.view(torch.int16) if o.dtype == torch.bfloat16 else o,
                                                    s1.view(torch.int16) if s1.dtype == torch.bfloat16 else s1)
    w, s, b = ws[2]
    ref = O.bf16_to_f32(xb).astype(np.float64) @ O.q4_dequant(w, s, b, O.F16).astype(np.float64).T
    assert _rel(to_np(outs[2]), ref) <= 1e-5


def test_q4_matmul_parts_rejects_bad_calls(hip):
    import qff
    from qff._lib import Q4Part, lib
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    w, s, b = _w_gpu(*synth.q4_weight(64, 128, seed=3), "f16")
    x = torch.zeros(1, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        qff.q4_matmul_parts(ctx, [], x)
    with pytest.raises(ValueError):
        qff.q4_matmul_parts(ctx, [(w, s, b)] * 9, x)
    arr = (Q4Part * 1)()
    arr[0] = Q4Part(w.data_ptr(), s.data_ptr(), b.data_ptr(), 0, x.data_ptr(), 0)   # rows = 0
    assert lib().qff_q4_matmul_parts(ctx.handle, None, arr, 1, 2, x.data_ptr(), 1, 128, 1) == -1
