"""Shared helpers for the GPU parity tests (inputs are drawn on the CPU with a
seeded generator and copied to the device, so CPU oracle and GPU see the same bytes)."""
import sys

import numpy as np
import torch

DEV = torch.device("cuda:0")


def announce(*parts) -> None:
    """Name the case before each GPU step (flushed, so a crash still shows it)."""
    print("[gpu-case]", *parts, flush=True)
    sys.stdout.flush()


def u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.uint8).numpy()


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def outlier_acts(M: int, K: int, g: torch.Generator) -> torch.Tensor:
    """benchmark cfg 0 activations: N(0,1) with 0.5% of channels scaled x20 (bf16)."""
    x = torch.randn(M, K, generator=g)
    cols = torch.randperm(K, generator=g)[: max(1, K // 200)]
    x[:, cols] *= 20
    return x.to(torch.bfloat16)
