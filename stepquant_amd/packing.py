"""Little-endian bit streams of 2/4/6/8-bit codes (stepquant/packing.py:6-22).

``n = 8 / gcd(bits, 8)`` codes form one word of ``n*bits/8`` bytes; code i of
a word occupies bits [i*bits, (i+1)*bits).  These streams are the
StateCodec storage format, not the pool page layout.  Works on tensors of any
device, like the reference.
"""
import math

import torch


def pack(codes, bits):
    if bits not in (2, 4, 6, 8):
        raise ValueError("supported code widths: 2, 4, 6, 8")
    flat = codes.reshape(-1).to(torch.int32)
    n = 8 // math.gcd(bits, 8)
    width = n * bits // 8
    flat = torch.nn.functional.pad(flat, (0, (-flat.numel()) % n)).reshape(-1, n)
    shifts = torch.arange(n, device=flat.device, dtype=torch.int32) * bits
    word = (flat << shifts).sum(-1, dtype=torch.int32)
    byte_shift = torch.arange(width, device=flat.device, dtype=torch.int32) * 8
    return ((word[:, None] >> byte_shift) & 255).to(torch.uint8).reshape(-1)


def unpack(data, bits, count):
    n = 8 // math.gcd(bits, 8)
    width = n * bits // 8
    shifts = torch.arange(width, device=data.device, dtype=torch.int64) * 8
    word = (data.to(torch.int64).reshape(-1, width) << shifts).sum(-1)
    codes = (word[:, None] >> (torch.arange(n, device=data.device) * bits)) & ((1 << bits) - 1)
    return codes.reshape(-1)[:count].to(torch.int16)
