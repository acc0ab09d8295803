"""Torch plumbing for the GPU tests: numpy <-> device tensors, bf16 bits."""
import sys

import numpy as np


def say(*args):
    """names the case before each GPU step, flushed, so a fault can be traced"""
    print("[gpu-case]", *args, flush=True)
    sys.stdout.flush()


def dev_f32(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


def dev_bf16(bits):
    """uint16 bf16 bit patterns -> torch.bfloat16 on the GPU"""
    import torch
    b = np.ascontiguousarray(bits, np.uint16)
    return torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).cuda()


def dev_u32(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.uint32).view(np.int32)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        bits = t.view(torch.int16).cpu().numpy().view(np.uint16)
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return t.cpu().numpy()


def host_bits(t):
    import torch
    torch.cuda.synchronize()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)
