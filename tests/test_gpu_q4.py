"""GPU parity of the affine-Q4 entry points.

qff_q4_dequant must be bit-exact with the closed form
(QwenQ4ActiveExpertStreamingRunner.swift:899-922) for f16 and bf16 scales.
qff_q4_matmul is checked against an fp64 product of the dequantized matrix.
Decode batches (<= 32 tokens) take the nibbles exactly and bf16 x exactly
(fp32 x as bf16 hi + lo pairs), so the relative Frobenius error must stay
<= 1e-5 (fp32 accumulation order only), against the exact fp32 x and against
the reference's own fp32 factored order (deltanet.metal:816-861). The
many-token GEMM (>= 33 tokens) runs on fp16 operands, W rounded once to
fp16 (2^8 (s q + b)) and x to fp16 after a per-token power-of-two shift:
each operand carries 11 significant bits, so its bar against the exact
product is rel <= 1e-3 (measured ~3e-4), for bf16 and fp32 x alike, and for
tokens whose magnitudes span 2^-40 .. 2^40 (dequantized weights keep 11 bits
for magnitudes 2^-22 .. 255, the range of real Q4 checkpoints).

qff_q4_norm_matmul_parts (RMSNorm, deltanet.metal:18-53, feeding the
products) is checked against a mirror of its arithmetic (inverse RMS in
fp64 applied to the row sums, x w_norm exact in fp32), rel <= 1e-5 for fp32
outputs of decode batches, and against the oracle's RMSNorm (pinned by the
reference's KAT) followed by an fp64 product: rel <= 1e-5 for decode
batches, <= 1e-3 for the GEMM (fp16 operands). Tokens carry different
scales so a norm taken from the wrong token shows. The residual store (y = residual + x W^T) must equal the
product plus the residual bit for bit with fp32 outputs, in place too."""
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


GEMM_MIN_BATCH = 33   # batches from here on take the fp16-operand GEMM


@pytest.mark.parametrize("rows,cols,batch", [(8192, 2048, 1), (512, 2048, 5), (4096, 2048, 16),
                                             (2048, 4096, 32), (100, 2048, 33), (32, 2048, 1),
                                             # 64-row workgroups (batch >= 2, >= 8192 rows), ragged end
                                             (8192, 2048, 2), (8200, 2048, 17), (9216, 2048, 32),
                                             # many-token GEMM path (batch >= 64), ragged tiles included
                                             (512, 2048, 64), (100, 2048, 300), (8192, 2048, 256),
                                             (2048, 4096, 130), (512, 2048, 8192),
                                             # 4096 columns, 2-16 tokens: the split-slice kernel
                                             (2048, 4096, 16), (100, 4096, 3), (2048, 4096, 2),
                                             # column counts that are not a multiple of 512
                                             (300, 576, 5), (200, 3136, 17), (64, 1088, 2),
                                             (8192, 1088, 4), (40, 192, 1), (40, 3136, 1)])
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
    assert _rel(to_np(y), ref) <= (1e-3 if batch >= GEMM_MIN_BATCH else 1e-5)


def test_q4_matmul_f32_activations_vs_reference_order(hip):
    import qff
    rows, cols = 2048, 4096
    w, s, b = synth.q4_weight(rows, cols, seed=99)
    x = np.random.default_rng(5).standard_normal((2, cols)).astype(np.float32)
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    y = qff.q4_matmul(ctx, *_w_gpu(w, s, b, "f16"), f32_tensor(x))
    y1 = qff.q4_matmul(ctx, *_w_gpu(w, s, b, "f16"), f32_tensor(x[:1]))
    yb = qff.q4_matmul(ctx, *_w_gpu(w, s, b, "f16"), f32_tensor(x), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    for m in range(2):
        ref = O.q4_matvec(w, s, b, x[m])
        assert _rel(to_np(y)[m], ref) <= 1e-5
        assert _rel(to_np(yb)[m], ref) <= 4e-3          # bf16 output rounding
    assert _rel(to_np(y1)[0], O.q4_matvec(w, s, b, x[0])) <= 1e-5   # the single-token kernel


def test_q4_gemv_f32_activations_64_row_workgroups(hip):
    """Decode batch over >= 8192 rows (four row tiles per workgroup) with fp32
    activations (hi + lo operands): the product matches the fp64 product of
    the exact x."""
    import qff
    rows, cols, batch = 8256, 2048, 9
    w, s, b = synth.q4_weight(rows, cols, seed=8)
    x = np.random.default_rng(9).standard_normal((batch, cols)).astype(np.float32)
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    y = qff.q4_matmul(ctx, *_w_gpu(w, s, b, "bf16"), f32_tensor(x))
    torch.cuda.synchronize()
    dense = O.q4_dequant(w, s, b, O.BF16).astype(np.float64)
    ref = x.astype(np.float64) @ dense.T
    assert _rel(to_np(y), ref) <= 1e-5


def test_q4_gemm_f32_activations(hip):
    """Many-token path with fp32 activations: the matrix cores take x as fp16
    after the per-token shift, so the product is the fp64 product of the
    exact fp32 x to the GEMM's fp16-operand bar."""
    import qff
    rows, cols, batch = 640, 2048, 96
    w, s, b = synth.q4_weight(rows, cols, seed=7)
    x = np.random.default_rng(6).standard_normal((batch, cols)).astype(np.float32)
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    y = qff.q4_matmul(ctx, *_w_gpu(w, s, b, "f16"), f32_tensor(x))
    torch.cuda.synchronize()
    dense = O.q4_dequant(w, s, b, O.F16).astype(np.float64)
    ref = x.astype(np.float64) @ dense.T
    assert _rel(to_np(y), ref) <= 1e-3


@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_q4_gemm_token_magnitudes(hip, xdt):
    """Tokens scaled by 2^-40 .. 2^40 (beyond fp16's range both ways, and an
    all-zero token): the per-token power-of-two shift keeps every token's x16
    in fp16's normal range, so each token's row of outputs meets the bar on
    its own, with no overflow and no flush to zero."""
    import qff
    rows, cols, batch = 300, 1024, 48
    w, s, b = synth.q4_weight(rows, cols, seed=21, sb_dtype="bf16")
    rng = np.random.default_rng(22)
    scale = 2.0 ** np.linspace(-40, 40, batch)
    x = (rng.standard_normal((batch, cols)) * scale[:, None]).astype(np.float32)
    x[5] = 0.0
    x[7, ::3] *= 1e-4   # a wide spread inside one token
    # the smallest tokens: 2^-120, and one made of fp32 subnormals (2^-136)
    scale[9], scale[11] = 2.0 ** -120, 2.0 ** -136
    x[9] = (rng.standard_normal(cols) * scale[9]).astype(np.float32)
    x[11] = (rng.standard_normal(cols) * scale[11]).astype(np.float32)
    if xdt == "bf16":
        x = O.round_bf16(x)
    xt = bf16_tensor(O.f32_to_bf16(x)) if xdt == "bf16" else f32_tensor(x)
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=64)
    y = to_np(qff.q4_matmul(ctx, *_w_gpu(w, s, b, "bf16"), xt))
    torch.cuda.synchronize()
    ref = x.astype(np.float64) @ O.q4_dequant(w, s, b, O.BF16).astype(np.float64).T
    assert np.all(np.isfinite(y))
    assert np.all(y[5] == 0.0)
    for m in range(batch):
        if m != 5:
            # compared at unit scale, so the smallest tokens' errors are not
            # lost below the helper's 1e-30 floor
            u = 1.0 / scale[m]
            assert _rel(y[m].astype(np.float64) * u, ref[m] * u) <= 1e-3, \
                f"token {m} (scale 2^{np.log2(scale[m]):.1f})"


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
    assert _rel(to_np(outs[2]), ref) <= (1e-3 if batch >= GEMM_MIN_BATCH else 1e-5)


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
    arr[0] = Q4Part(w.data_ptr(), s.data_ptr(), b.data_ptr(), 0, x.data_ptr(), 0, None)   # rows = 0
    assert lib().qff_q4_matmul_parts(ctx.handle, None, arr, 1, 2, x.data_ptr(), 1, 128, 1) == -1


def _norm_mirror(x, wn, eps):
    """x w_norm as the product takes it (fp32 multiply) and the inverse RMS
    of each token in fp64."""
    x64 = x.astype(np.float64)
    r = 1.0 / np.sqrt((x64 * x64).mean(axis=1) + eps)
    xw = (x.astype(np.float32) * wn.astype(np.float32)).astype(np.float32)
    return xw.astype(np.float64), r


@pytest.mark.parametrize("batch,cols,xdt,ndt", [(1, 2048, "bf16", "f32"), (1, 4096, "f32", "bf16"),
                                                (3, 2048, "bf16", "bf16"), (16, 2048, "bf16", "f32"),
                                                (32, 4096, "f32", "f32"), (40, 2048, "bf16", "f32"),
                                                (300, 2048, "f32", "bf16"), (1, 128, "bf16", "f32")])
def test_q4_norm_matmul_parts(hip, batch, cols, xdt, ndt):
    import qff
    print(f"q4_norm_matmul_parts batch={batch} cols={cols} x={xdt} norm={ndt}", flush=True)
    rng = np.random.default_rng(7 * batch + cols)
    scale = 2.0 ** (np.arange(batch) % 5 - 2)
    x = (rng.standard_normal((batch, cols)) * scale[:, None]).astype(np.float32)
    if xdt == "bf16":
        x = O.round_bf16(x)
    wn = (1.0 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    if ndt == "bf16":
        wn = O.round_bf16(wn)
    eps = 1e-6
    shapes = [(1056, torch.bfloat16), (32, torch.float32), (100, torch.float32)]
    ws = [synth.q4_weight(r, cols, seed=r + batch) for r, _ in shapes]
    parts = [_w_gpu(w, s, b, "f16") for w, s, b in ws]
    xt = bf16_tensor(O.f32_to_bf16(x)) if xdt == "bf16" else f32_tensor(x)
    nt = bf16_tensor(O.f32_to_bf16(wn)) if ndt == "bf16" else f32_tensor(wn)
    ctx = qff.Context(max_batch=32, max_ctx=64, max_prefill_tokens=512)
    outs = qff.q4_norm_matmul_parts(ctx, parts, xt, nt, eps, out_dtypes=[dt for _, dt in shapes])
    torch.cuda.synchronize()
    gemm = batch >= GEMM_MIN_BATCH
    xq, r = _norm_mirror(x, wn, eps)
    xn = np.stack([O.rmsnorm(x[m], wn, eps, prec=64) for m in range(batch)]).astype(np.float64)
    bar = 1e-3 if gemm else 1e-5
    for o, (w, s, b), (_, dt) in zip(outs, ws, shapes):
        dense = O.q4_dequant(w, s, b, O.F16).astype(np.float64)
        got = to_np(o)
        assert _rel(got, r[:, None] * (xq @ dense.T)) <= (bar if dt == torch.float32 else 4e-3)
        assert _rel(got, xn @ dense.T) <= (bar if dt == torch.float32 else 4e-3)


@pytest.mark.parametrize("batch", [1, 7, 33])
def test_q4_matmul_parts_residual(hip, batch):
    """y = residual + x W^T: fp32 outputs equal the plain product plus the
    residual bit for bit (one fp32 add), also when the residual is y itself;
    bf16 outputs match the fp64 sum."""
    import qff
    print(f"q4_matmul_parts residual batch={batch}", flush=True)
    cols, rows = 2048, 640
    w, s, b = synth.q4_weight(rows, cols, seed=5 + batch, sb_dtype="bf16")
    part = _w_gpu(w, s, b, "bf16")
    rng = np.random.default_rng(batch)
    xb = O.f32_to_bf16(rng.standard_normal((batch, cols)).astype(np.float32))
    x = bf16_tensor(xb)
    res = f32_tensor(rng.standard_normal((batch, rows)).astype(np.float32) * 30)
    ctx = qff.Context(max_batch=32, max_ctx=64, max_prefill_tokens=64)
    plain = qff.q4_matmul_parts(ctx, [part], x)[0]
    added = qff.q4_matmul_parts(ctx, [part], x, residuals=[res])[0]
    inplace = res.clone()
    qff.q4_matmul_parts(ctx, [part], x, outs=[inplace], residuals=[inplace])
    res_bf = res.to(torch.bfloat16)
    out_bf = qff.q4_matmul_parts(ctx, [part], x, out_dtypes=[torch.bfloat16], residuals=[res_bf])[0]
    torch.cuda.synchronize()
    assert torch.equal(added, plain + res)
    assert torch.equal(inplace, added)
    ref = to_np(res_bf).astype(np.float64) + O.bf16_to_f32(xb).astype(np.float64) @ \
        O.q4_dequant(w, s, b, O.BF16).astype(np.float64).T
    assert _rel(to_np(out_bf), ref) <= 4e-3


@pytest.mark.parametrize("batch", [2, 9, 16])
def test_q4_matmul_parts_4096_cols_f32_x_residual(hip, batch):
    """The out-projection shape (4096 columns, 2-16 tokens, fp32 x, a residual
    added in place) through the split-slice kernel and its reduction launch:
    two parts with a ragged row tile, fp32 and bf16 outputs, against fp64
    products of the fp32 x; called twice so the second call reuses the
    workspace the first one filled."""
    import qff
    print(f"q4_matmul_parts 4096 cols batch={batch}", flush=True)
    cols = 4096
    shapes = [(2048, torch.float32), (100, torch.bfloat16)]
    ws = [synth.q4_weight(r, cols, seed=r + 11 * batch) for r, _ in shapes]
    parts = [_w_gpu(w, s, b, "f16") for w, s, b in ws]
    rng = np.random.default_rng(40 + batch)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    res0 = (rng.standard_normal((batch, 2048)) * 30).astype(np.float32)
    ctx = qff.Context(max_batch=32, max_ctx=64, max_prefill_tokens=64)
    for _ in range(2):
        y0 = f32_tensor(res0)
        y1 = torch.empty(batch, 100, dtype=torch.bfloat16, device=DEV)
        outs = qff.q4_matmul_parts(ctx, parts, f32_tensor(x), outs=[y0, y1], residuals=[y0, None])
        torch.cuda.synchronize()
        for i, ((w, s, b), (_, dt)) in enumerate(zip(ws, shapes)):
            ref = x.astype(np.float64) @ O.q4_dequant(w, s, b, O.F16).astype(np.float64).T
            if i == 0:
                ref = ref + res0.astype(np.float64)
            assert _rel(to_np(outs[i]), ref) <= (1e-5 if dt == torch.float32 else 4e-3)


def test_q4_norm_matmul_parts_rejects_bad_calls(hip):
    import qff
    from qff._lib import Q4Part, lib
    ctx = qff.Context(max_batch=1, max_ctx=64, max_prefill_tokens=1)
    w, s, b = _w_gpu(*synth.q4_weight(64, 128, seed=3), "f16")
    x = torch.zeros(1, 128, dtype=torch.bfloat16, device=DEV)
    y = torch.zeros(1, 64, device=DEV)
    arr = (Q4Part * 1)()
    arr[0] = Q4Part(w.data_ptr(), s.data_ptr(), b.data_ptr(), 64, y.data_ptr(), 0, None)
    nw = torch.ones(128, device=DEV)
    L = lib()
    assert L.qff_q4_norm_matmul_parts(ctx.handle, None, arr, 1, 2, x.data_ptr(), 1, None, 0, 1e-6, 128, 1) == -1
    assert L.qff_q4_norm_matmul_parts(ctx.handle, None, arr, 1, 2, x.data_ptr(), 1, nw.data_ptr(), 0, -1.0,
                                      128, 1) == -1
    assert L.qff_q4_norm_matmul_parts(ctx.handle, None, arr, 1, 2, x.data_ptr(), 1, nw.data_ptr(), 0, 1e-6,
                                      96, 1) == -2
    with pytest.raises(ValueError):
        qff.q4_norm_matmul_parts(ctx, [(w, s, b)], x, torch.ones(64, device=DEV))


@pytest.mark.parametrize("batch", [16, 200])
def test_q4_matmul_parts_graph_replay(hip, batch):
    """The three GQA in-projections (8192 + 512 + 512 rows x 2048) in one
    call, captured in a HIP graph and replayed three times with an eager
    product of another batch on the same context between replays (which
    rewrites the context's x16 and token factors, or the split's partials):
    every replay equals an eager call on the same inputs, bit for bit.
    batch 16 runs the decode-shaped kernel, 200 the prefill GEMM."""
    import qff
    print(f"q4_matmul_parts graph replay batch={batch}", flush=True)
    cols = 2048
    ws = [synth.q4_weight(r, cols, seed=500 + r) for r in (8192, 512, 512)]
    parts = [_w_gpu(w, s, b, "f16") for w, s, b in ws]
    rng = np.random.default_rng(600 + batch)
    x = bf16_tensor(O.f32_to_bf16(rng.standard_normal((batch, cols)).astype(np.float32)))
    x2 = bf16_tensor(O.f32_to_bf16(rng.standard_normal((40, cols)).astype(np.float32)))
    ctx = qff.Context(max_batch=32, max_ctx=64, max_prefill_tokens=256)
    ref = [o.clone() for o in qff.q4_matmul_parts(ctx, parts, x)]
    torch.cuda.synchronize()
    outs = [torch.empty_like(o) for o in ref]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        qff.q4_matmul_parts(ctx, parts, x, outs=outs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        qff.q4_matmul_parts(ctx, parts, x, outs=outs)
    for rep in range(3):
        print(f"q4_matmul_parts graph replay {rep}", flush=True)
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o.view(torch.int16), r.view(torch.int16)), f"replay {rep}"
        qff.q4_matmul_parts(ctx, parts, x2)
        torch.cuda.synchronize()
