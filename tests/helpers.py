"""Shared helpers for the tests: numpy <-> torch for bf16 bit patterns, GPU launch wrappers."""
import numpy as np
import torch


def to_dev_bf16(bits: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(dev)


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def dev_inputs(inp, dev):
    """(x bf16 [M,K], w_t int8 [K,N] stride (1,K), s fp32 [N]) on dev from oracle.Inputs."""
    x = to_dev_bf16(inp.x, dev)
    w = torch.from_numpy(inp.w).to(dev)
    s = torch.from_numpy(inp.s).to(dev)
    return x, w.t(), s
