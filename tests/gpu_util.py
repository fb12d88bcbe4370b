"""Helpers shared by the GPU parity tests: numpy <-> torch on cuda:0 and the
tolerance rules written once."""
import numpy as np
import torch

from oracle import oracle as O

DEV = "cuda:0"


def bf16_tensor(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def f16_tensor(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.float16).to(DEV)


def f32_tensor(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(DEV)


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return O.bf16_to_f32(t.view(torch.int16).numpy().view(np.uint16))
    return t.float().numpy()


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |x| (8 significant bits)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def assert_bf16_output_close(gpu: np.ndarray, ref: np.ndarray, atol: float = 2e-2):
    """bf16 outputs: max-abs error <= 2e-2 against the fp32 reference, where a
    value whose bf16 spacing exceeds 2e-2 (|x| >= 4) may also sit one bf16
    ulp away -- rounding to the output dtype alone can cost that much."""
    err = np.abs(gpu.astype(np.float64) - ref.astype(np.float64))
    lim = np.maximum(atol, bf16_ulp(ref))
    bad = err > lim
    assert not bad.any(), (f"{bad.sum()} of {bad.size} outside tolerance; worst err "
                           f"{err.max():.4g} at ref {ref.reshape(-1)[err.argmax()]:.4g}")


def assert_f32_output_close(gpu: np.ndarray, ref: np.ndarray, atol: float = 2e-2):
    err = np.max(np.abs(gpu.astype(np.float64) - ref.astype(np.float64)))
    assert err <= atol, f"max-abs error {err:.4g} > {atol}"


def state_rel_err(gpu: np.ndarray, ref: np.ndarray) -> float:
    """Per-head Frobenius relative error of fp32 state [.., 32, 128, 128],
    max over heads."""
    g = gpu.reshape(-1, 128 * 128).astype(np.float64)
    r = ref.reshape(-1, 128 * 128).astype(np.float64)
    return float(np.max(np.linalg.norm(g - r, axis=1) / np.maximum(np.linalg.norm(r, axis=1), 1e-30)))
