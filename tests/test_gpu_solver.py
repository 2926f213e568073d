"""ditk_solver_step (fused CFG combine + UniPC / FlowMatch-Euler) against the
float64 oracle over whole trajectories.  Tolerance: relative error <= 1e-5 of
the fp32 kernel against float64 (coefficients are float64 on the host, cast to
fp32)."""
import numpy as np
import pytest
import torch

from oracle import solver as osv

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


@pytest.mark.parametrize("steps,order,cfg", [(10, 2, True), (6, 1, True), (4, 2, False)])
def test_unipc_trajectory_matches_oracle(steps, order, cfg):
    from ditserve_amd.solver import UniPCFlowScheduler
    rng = np.random.default_rng(steps)
    shape = (16, 3, 10, 18)
    sched = UniPCFlowScheduler(flow_shift=3.0, solver_order=order)
    sched.set_timesteps(steps)
    ref = osv.UniPCFlowOracle(osv.unipc_flow_sigmas(steps, 3.0)[0], solver_order=order)
    x = rng.standard_normal(shape)
    xd = torch.tensor(x, dtype=torch.float32, device=DEV)
    xr = x.copy()
    for i in range(steps):
        c, u = rng.standard_normal(shape), rng.standard_normal(shape)
        cd = torch.tensor(c, dtype=torch.float32, device=DEV)
        ud = torch.tensor(u, dtype=torch.float32, device=DEV) if cfg else None
        xd = sched.step(cd, sched.timesteps[i], xd, uncond=ud, guidance=5.0)[0]
        xr = ref.step(osv.cfg(c, u if cfg else None, 5.0), xr)
        assert _rel(xd.cpu().double().numpy(), xr) < 1e-5, f"step {i}"
    assert sched.step_index == steps


def test_flowmatch_euler_trajectory_matches_oracle():
    from ditserve_amd.solver import FlowMatchEulerScheduler
    rng = np.random.default_rng(3)
    sched = FlowMatchEulerScheduler(shift=3.0)
    sched.set_timesteps(12)
    ref = osv.FlowMatchEulerOracle(osv.flowmatch_sigmas(12, 3.0)[0])
    x = rng.standard_normal((16, 64, 64))
    xd = torch.tensor(x, dtype=torch.float32, device=DEV)
    for i in range(12):
        c, u = rng.standard_normal(x.shape), rng.standard_normal(x.shape)
        xd = sched.step(torch.tensor(c, dtype=torch.float32, device=DEV), sched.timesteps[i], xd,
                        uncond=torch.tensor(u, dtype=torch.float32, device=DEV), guidance=7.0)[0]
        x = ref.step(osv.cfg(c, u, 7.0), x)
        assert _rel(xd.cpu().double().numpy(), x) < 1e-5, f"step {i}"


def test_solver_step_in_place_and_odd_sizes():
    """x_next aliasing x, a length that is not a multiple of the block, and a
    null-history call rejected when its coefficient needs the buffer."""
    from ditserve_amd import ops
    from ditserve_amd._lib import DitkError
    n = 1000003
    x = torch.randn(n, device=DEV)
    c = torch.randn(n, device=DEV)
    want = (x + 0.25 * c).cpu()
    coef = [1.0, 0.0, 1.0, 0.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.25]
    ops.solver_step(x, c, coef, x_next=x)
    torch.testing.assert_close(x.cpu(), want, rtol=1e-6, atol=1e-6)
    with pytest.raises(DitkError):
        ops.solver_step(x, c, [1.0, 0.5, 0.0, 1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0])
