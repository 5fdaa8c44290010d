"""Helpers for the GPU tests: device buffers (torch is used only to allocate
device memory) and a session context on cuda:0."""
import ctypes

import numpy as np

import ggnpu_amd.lib as gl

PAD = 256


def torch_mod():
    import torch
    return torch


def dev(a):
    """numpy array -> contiguous device tensor (uint8 views get PAD bytes of
    zeroed tail so realigning loads stay inside the allocation)."""
    torch = torch_mod()
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint8:
        t = torch.zeros(a.size + PAD, dtype=torch.uint8, device="cuda")
        t[: a.size].copy_(torch.from_numpy(a.reshape(-1)))
        return t
    return torch.from_numpy(a).to("cuda")


def empty(shape, dtype):
    torch = torch_mod()
    return torch.empty(shape, dtype=dtype, device="cuda")


def host(t):
    torch = torch_mod()
    torch.cuda.synchronize()
    return t.cpu().numpy()


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def stream_handle():
    torch = torch_mod()
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
