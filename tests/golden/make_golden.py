"""Write golden vectors for fit_state and StateCodec from the reference.

This script runs the reference's pure-PyTorch quantiser
(stepquant/quantization.py:54-152, which imports stepquant/packing.py) in the
build container only, because the bit-exact output of fit_state depends on
PyTorch's CPU float32 summation order and nothing short of running it pins
that.  The vectors (inputs and outputs) are saved to
tests/golden/fit_state_vectors.npz; nothing from the reference is copied.

Usage:  python tests/golden/make_golden.py [/root/reference]
"""
import hashlib
import json
import os
import sys

import numpy as np
import torch

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
sys.path.insert(0, REF)
from stepquant.quantization import QuantizationPlan, StateCodec, fit_state  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fit_state_vectors.npz")


def make_cases():
    g = torch.Generator().manual_seed(20261201)

    def randn(*shape, std=1.0):
        return torch.randn(*shape, generator=g) * std

    def rand(*shape):
        return torch.rand(*shape, generator=g)

    cases = {}
    # CPU config of the benchmark: GDN, B=2, H=4, dk=dv=128, state ~ N(0, 0.05^2),
    # per-head widths from {4,6,8} averaging 6 plus one FP16 pivot head.
    cases["c_config_gdn"] = dict(arch="gdn", bits=torch.tensor([6, 4, 8, 16])[:, None].expand(4, 128),
                                 impact=rand(4, 128) + .5, group=32, x=randn(2, 4, 128, 128, std=.05))
    cases["c_config_gdn_uniform6"] = dict(arch="gdn", bits=torch.full((4, 128), 6),
                                          impact=torch.ones(4, 128), group=32,
                                          x=randn(2, 4, 128, 128, std=.05))
    # GDN INT2 heads with value-group row scales.
    cases["gdn_two_bit_g32"] = dict(arch="gdn", bits=torch.tensor([2, 6, 2])[:, None].expand(3, 128),
                                    impact=rand(3, 128) + .5, group=32, x=randn(1, 3, 128, 128, std=.05))
    # Reference test_core.py:46-64 shapes: widths 2..16 per head, V=16, group 4.
    cases["gdn_mixed_v16_g4"] = dict(arch="gdn", bits=torch.tensor([2, 4, 6, 8, 16])[:, None].expand(5, 8),
                                     impact=rand(5, 8) + .2, group=4, x=randn(2, 5, 8, 16))
    cases["kda_mixed_v16"] = dict(arch="kda", bits=torch.tensor([2, 4, 6, 8, 16])[:, None].expand(5, 8).T,
                                  impact=rand(8, 5) + .2, group=32, x=randn(2, 8, 5, 16))
    # KDA per-row widths {4,6,8} with FP16 pivot rows, full head size.
    kb = torch.tensor([4, 6, 8]).repeat(2, 43)[:, :128].clone()
    kb[:, ::17] = 16
    cases["kda_mixed_128"] = dict(arch="kda", bits=kb, impact=torch.linspace(.25, 2., 256).reshape(2, 128),
                                  group=32, x=randn(2, 2, 128, 128, std=.1))
    # Half-aligned KDA pages (reference test_kernel_edges.py:10-30).
    for v in (4, 32):
        cases[f"kda_edges_v{v}"] = dict(arch="kda", bits=torch.tensor([[2, 4, 8, 16]]),
                                        impact=torch.ones(1, 4), group=32, x=randn(3, 1, 4, v))
    # Narrow value dims take the interleaved (ilp) key-axis order in torch.
    cases["gdn_v8_k4"] = dict(arch="gdn", bits=torch.tensor([4, 6, 8, 2])[:, None].expand(4, 4),
                              impact=rand(4, 4) + .5, group=4, x=randn(2, 4, 4, 8))
    cases["gdn_v32_k32"] = dict(arch="gdn", bits=torch.tensor([6, 2, 4, 8, 16])[:, None].expand(5, 32),
                                impact=rand(5, 32) + .5, group=32, x=randn(2, 5, 32, 32, std=.3))
    # Zero state and scale extremes (clamps at 2^-24 and large magnitudes).
    cases["zero_state"] = dict(arch="gdn", bits=torch.tensor([6, 2])[:, None].expand(2, 16),
                               impact=torch.ones(2, 16), group=8, x=torch.zeros(1, 2, 16, 32))
    xe = randn(1, 2, 16, 32)
    xe[0, 0, :4] *= 1e4
    xe[0, 0, 4:8] *= 1e-12
    xe[0, 1, 8:12] = 0
    xe[0, 1, 12] *= 1e-30
    cases["scale_extremes"] = dict(arch="kda", bits=torch.tensor([[6] * 8 + [8, 4, 2, 16] * 2] * 2),
                                   impact=rand(2, 16) + .1, group=32, x=xe)
    # KDA pivots excluded from the shared column fit (test_core.py:97-106).
    xp = randn(1, 1, 5, 32)
    yp = xp.clone()
    yp[:, :, 4] *= 1000
    for name, val in (("kda_pivot_a", xp), ("kda_pivot_b", yp)):
        cases[name] = dict(arch="kda", bits=torch.tensor([[2, 4, 6, 8, 16]]), impact=torch.ones(1, 5),
                           group=32, x=val)
    return cases


def sha(t):
    return hashlib.sha256(np.ascontiguousarray(t).tobytes()).hexdigest()


def main():
    arrays = {}
    meta = {"torch": torch.__version__, "cpu_capability": torch.backends.cpu.get_cpu_capability(),
            "threads": torch.get_num_threads(), "cases": {}}
    for name, case in make_cases().items():
        bits = case["bits"].contiguous().to(torch.int64)
        impact = case["impact"].contiguous().float()
        plan = QuantizationPlan(case["arch"], bits, impact, case["group"])
        x = case["x"].contiguous().float()
        z, r, c, r2, recon = fit_state(x, plan)
        packed = StateCodec(plan).encode(x)
        arrays[f"{name}/x"] = x.numpy()
        arrays[f"{name}/bits"] = bits.numpy().astype(np.int32)
        arrays[f"{name}/impact"] = impact.numpy()
        arrays[f"{name}/z"] = z.numpy().astype(np.int8)
        arrays[f"{name}/r"] = r.numpy().view(np.uint16)
        arrays[f"{name}/c"] = c.numpy().view(np.uint16)
        if r2 is not None:
            arrays[f"{name}/r2"] = r2.numpy().view(np.uint16)
        small = x.numel() <= 65536
        if small:
            arrays[f"{name}/recon"] = recon.numpy()
            for b, stream in packed.codes.items():
                arrays[f"{name}/codec{b}"] = stream.numpy()
            arrays[f"{name}/codec_pivots"] = packed.pivots.numpy().view(np.uint16)
        meta["cases"][name] = dict(
            arch=case["arch"], group=case["group"], shape=list(x.shape),
            recon_sha256=sha(recon.numpy()),
            codec_sha256={str(b): sha(s.numpy()) for b, s in packed.codes.items()},
            codec_rows_sha256=sha(packed.rows.numpy().view(np.uint16)),
            codec_columns_sha256=sha(packed.columns.numpy().view(np.uint16)),
            codec_pivots_sha256=sha(packed.pivots.numpy().view(np.uint16)),
            codec_nbytes=int(packed.nbytes))
    arrays["meta"] = np.frombuffer(json.dumps(meta, sort_keys=True).encode(), np.uint8)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(meta['cases'])} cases)")


if __name__ == "__main__":
    main()
