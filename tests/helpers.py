"""Shared helpers of the GPU parity tests: seeded inputs of the BitLinear
configurations and bf16 bit-pattern transfers between numpy and torch."""

import numpy as np


def dev():
    import torch

    return torch.device("cuda:0")


def to_dev_bf16(bits: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev()).view(torch.bfloat16)


def bits_of(t) -> np.ndarray:
    import torch

    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def to_dev(arr: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(arr)).to(dev())


def activations(orc, m, k, seed, outliers=True, scale=1.0):
    """bf16 bits of x ~ N(0, 1) with 1 % of the channels (fixed by the seed) x20."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32) * scale
    if outliers:
        cols = rng.choice(k, max(1, k // 100), replace=False)
        x[:, cols] *= 20.0
    return orc.f32_to_bf16(x)


def latent(out_f, in_f, seed, std=0.02):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((out_f, in_f)) * std).astype(np.float32)


def gamma(orc, n, seed, std=0.1):
    rng = np.random.default_rng(seed)
    return orc.f32_to_bf16((1.0 + std * rng.standard_normal(n)).astype(np.float32))


def ternary(k, n, seed):
    rng = np.random.default_rng(seed)
    return rng.choice([-1, 0, 1], size=(k, n)).astype(np.int8)


def xa_to_rowmajor(xa: np.ndarray, m: int, k: int) -> np.ndarray:
    """Decode the blocked activation layout (32-row blocks, 128-column
    superblocks, 16 bytes per lane) back to [m, k] int8."""
    ks = (k + 127) // 128
    mb = (m + 31) // 32
    a = xa.view(np.int8).reshape(mb, ks, 4, 2, 32, 16)  # mb, ks, q, half, row, byte
    full = a.transpose(0, 4, 1, 2, 3, 5).reshape(mb * 32, ks * 128)
    return full[:m, :k], full


def rowmajor_to_xa(q: np.ndarray) -> np.ndarray:
    """[m, k] int8 -> blocked activation bytes (inverse of xa_to_rowmajor)."""
    m, k = q.shape
    ks = (k + 127) // 128
    mb = (m + 31) // 32
    full = np.zeros((mb * 32, ks * 128), np.int8)
    full[:m, :k] = q
    return np.ascontiguousarray(full.reshape(mb, 32, ks, 4, 2, 16).transpose(0, 2, 3, 4, 1, 5)).reshape(-1).view(np.uint8)
