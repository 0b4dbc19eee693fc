"""Host <-> device helpers shared by the GPU tests (numpy arrays from the oracle,
torch tensors as device memory)."""
import sys

import numpy as np
import torch


def note(msg: str) -> None:
    """Name the case on stdout before a GPU step (survives a crashed box)."""
    print(msg, flush=True)
    sys.stdout.flush()


def dev_h(a: np.ndarray) -> torch.Tensor:
    """uint16 fp16 bit patterns -> fp16 device tensor (same shape)."""
    a = np.ascontiguousarray(a, np.uint16)
    return torch.from_numpy(a.view(np.int16)).cuda().view(torch.float16)


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host_h(t: torch.Tensor) -> np.ndarray:
    """fp16 device tensor -> uint16 bit patterns."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def d_pos_for(seq: int) -> torch.Tensor:
    return torch.tensor([seq - 1], dtype=torch.int32, device="cuda")


def abs_err(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))
