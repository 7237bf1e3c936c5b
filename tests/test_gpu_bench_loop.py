"""bench.py's training loop, which launches step n + 1 before it reads step n's
finite flag (LaggedSteps), against the same steps in the reference loop's order
(train.py:649-672: read the flag, then step the optimizers; moe_train_step_sync):
identical parameters, optimizer state and step counts, through a non-finite
step (skipped) and a routing that overflows the static slot capacity
(recomputed with exact bucketing).  The lagged loop gates SparseAdam on the
device (step count and bias corrections on the GPU) and keeps the dynamic loss
scale on the device (DeviceLossScale); the synchronous loop steps SparseAdam
from the host and moves the loss scale by the reference's host schedule
(train.py:661-677: halve on a skipped step, double every SCALE_UP_EVERY good
steps, here 2 so that 6 steps double it twice).  Both refresh the overlay tables of the fused GEMMs
from the masters after each applied step, so every forward after the first
multiplies trained weights."""
import pytest
import torch

import bench

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _build(dev, zero_router):
    L = bench.build_moe(dev, T=96, H=256, I=128, E=8, k=2, seed=5, scale_up_every=2)
    if zero_router:
        # every expert ties for every token: 96 * 8 pairs against 96 * 3 static slots
        with torch.no_grad():
            L["router_w"].zero_()
    return L


def _set_dy(L, dy0, step, nan_step):
    with torch.no_grad():
        L["dy"].copy_(dy0)
        if step == nan_step:
            L["dy"][3, 5] = float("nan")


def _state(L):
    opt = L["opt"]
    out = {"router_w": L["router_w"].detach().clone(), "sgd_buf": L["sgd"]._buf[0].clone(), "adam_step": opt.step_count}
    for n in opt._active_ids:
        out[f"master:{n}"] = opt._named[n].detach().clone()
        out[f"m:{n}"] = opt._m[n].clone()
        out[f"v:{n}"] = opt._v[n].clone()
    return out


@pytest.mark.parametrize("zero_router,nan_step", [(False, 2), (True, 3)])
def test_lagged_loop_matches_sync_loop(gpu_device, zero_router, nan_step):
    _say(f"bench loop: lagged flag reads vs synchronous, 6 steps, zero_router={zero_router} nan_step={nan_step}")
    steps = 6
    A = _build(gpu_device, zero_router)
    dy0 = A["dy"].clone()
    finite_sync = []
    for s in range(steps):
        _set_dy(A, dy0, s, nan_step)
        finite_sync.append(bench.moe_train_step_sync(A))
    torch.cuda.synchronize()
    want = _state(A)

    B = _build(gpu_device, zero_router)
    loop = bench.LaggedSteps(B)
    for s in range(steps):
        _set_dy(B, dy0, s, nan_step)
        loop.step()
    loop.flush()
    torch.cuda.synchronize()
    got = _state(B)

    assert finite_sync.count(False) == 1 and not finite_sync[nan_step]
    assert loop.applied == steps - 1 and loop.skipped == 1
    assert loop.recomputed == A.get("recomputed", 0)
    assert (loop.recomputed >= 1) == zero_router
    assert got["adam_step"] == want["adam_step"] == steps - 1
    hsc = A["host_scale"]
    # 5 good steps at every 2: doubled twice, halved once -> 8192
    assert (hsc["loss_scale"], hsc["good_streak"], hsc["n_skipped"]) == (8192.0, steps - 1, 1)
    assert B["scaler"].state_dict() == {"loss_scale": hsc["loss_scale"], "good_streak": hsc["good_streak"],
                                        "n_skipped": hsc["n_skipped"]}
    for key in want:
        if key == "adam_step":
            continue
        assert torch.equal(got[key], want[key]), f"{key} differs between the lagged and the synchronous loop"
