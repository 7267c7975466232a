"""Helpers shared by the GPU parity tests (numpy <-> device tensors with byte-exact views)."""
import numpy as np
import torch

DEV = torch.device("cuda:0")

_VIEW = {np.uint8: torch.uint8, np.int8: torch.int8, np.uint16: torch.int16, np.int16: torch.int16,
         np.uint32: torch.int32, np.int32: torch.int32, np.float32: torch.float32}


def d(a: np.ndarray) -> torch.Tensor:
    """numpy array -> device tensor holding the same bytes (uint16 / uint32 carried as int16 / int32)."""
    a = np.ascontiguousarray(a)
    t = _VIEW[a.dtype.type]
    signed = {np.uint16: np.int16, np.uint32: np.int32}.get(a.dtype.type, a.dtype.type)
    return torch.from_numpy(a.view(signed)).to(DEV)


def h(t: torch.Tensor, dtype) -> np.ndarray:
    """device tensor -> numpy array of `dtype` over the same bytes."""
    torch.cuda.synchronize()
    return t.detach().cpu().contiguous().numpy().view(dtype)


def filled(shape, value, dtype=torch.uint8) -> torch.Tensor:
    return torch.full(shape, value, dtype=dtype, device=DEV)


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> uint16 numpy bits."""
    return x.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
