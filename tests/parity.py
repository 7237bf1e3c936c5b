"""Error measures shared by the GPU parity tests.

normwise rel = max|got - ref| / max|ref|, with the bars of every GPU test here
(1e-2 bf16, 2e-3 fp16); beside it the elementwise relative error
|got - ref| / max(|ref|, 0.01 rms(ref)) at its 99th percentile, bounded
loosely (5e-2 bf16, 1e-2 fp16) so that a few wrong elements cannot hide under
the normwise bar.
"""
import numpy as np
import torch

TOL = {torch.bfloat16: 1e-2, torch.float16: 2e-3}
P99 = {torch.bfloat16: 5e-2, torch.float16: 1e-2}


def errs(got, ref):
    """(normwise rel, elementwise p99 rel) of got against ref."""
    got = got.detach().float().cpu().reshape(-1)
    ref = ref.detach().float().cpu().reshape(-1)
    scale = float(ref.abs().max())
    assert scale > 0, "reference is all zeros"
    norm = float((got - ref).abs().max()) / scale
    floor = 0.01 * float(ref.pow(2).mean().sqrt())
    r = ((got - ref).abs() / ref.abs().clamp_min(max(floor, 1e-30))).numpy()
    return norm, float(np.percentile(r, 99))


def check(name, got, ref, dtype, report=None, say=None):
    """Assert both bars for `dtype`; record and print the two figures."""
    norm, p99 = errs(got, ref)
    if report is not None:
        report[name] = (norm, p99)
    msg = f"  {name}: normwise {norm:.2e} (bar {TOL[dtype]:.0e}), p99 elementwise {p99:.2e} (bar {P99[dtype]:.0e})"
    (say or (lambda m: print(f"[gpu-case] {m}", flush=True)))(msg)
    assert norm <= TOL[dtype], f"{name}: normwise {norm:.3e} > {TOL[dtype]}"
    assert p99 <= P99[dtype], f"{name}: p99 elementwise {p99:.3e} > {P99[dtype]}"
