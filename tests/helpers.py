"""Shared helpers for the parity tests (oracle side and device side)."""
import numpy as np
import torch

from oracle import oracle as O


def dev():
    if not torch.cuda.is_available():
        raise RuntimeError("GPU test selected but no HIP device is visible")
    return torch.device("cuda:0")


def make_plan(arch, bits, impact=None, group=32, seed=0):
    bits = np.asarray(bits, np.int32)
    if impact is None:
        impact = np.random.default_rng(seed).random(bits.shape).astype(np.float32) + .5
    return O.Plan(arch, bits, np.asarray(impact, np.float32), group)


def device_plan(oplan):
    from stepquant_amd.quantization import QuantizationPlan
    d = dev()
    return QuantizationPlan(oplan.architecture, torch.from_numpy(oplan.bits.astype(np.int64)).to(d),
                            torch.from_numpy(oplan.impact).to(d), oplan.value_group_size)


def page_codes(pages, slots, oplan, lay, V):
    """Integer codes [B,H,K,V] (pivots: fp16 bits) read from page bytes."""
    H, K = oplan.bits.shape
    tile = min(4 if oplan.kda else 16, V)
    out = np.zeros((len(slots), H, K, V), np.int64)
    for bi, s in enumerate(slots):
        if s <= 0:
            continue
        page = pages[s]
        bitsarr = np.unpackbits(page, bitorder="little")
        for h in range(H):
            stride = lay.offsets[H * K + h]
            for i in range(K):
                w = int(oplan.bits[h, i])
                off = int(lay.offsets[h * K + i])
                j = np.arange(V)
                start = (off + (j // tile) * stride) * 8 + (j % tile) * w
                idx = start[:, None] + np.arange(w)[None, :]
                out[bi, h, i] = (bitsarr[idx] << np.arange(w)[None, :]).sum(-1)
    return out


def scales(pages, slots, oplan, lay, V):
    """(row scales per row (and group), column scales) as float32 from pages."""
    H, K = oplan.bits.shape
    rs, cs = [], []
    for s in slots:
        page = pages[s]
        r = [page[o:o + 2 * (V // oplan.value_group_size if (not oplan.kda and oplan.bits[i // K, 0] == 2) else 1)]
             .view(np.float16).astype(np.float32) if o >= 0 else np.zeros(0, np.float32)
             for i, o in enumerate(lay.rows)]
        c = [page[o:o + 2 * V].view(np.float16).astype(np.float32) if o >= 0 else np.zeros(V, np.float32)
             for o in lay.columns]
        rs.append(r)
        cs.append(np.stack(c))
    return rs, np.stack(cs)
