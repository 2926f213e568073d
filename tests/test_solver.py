"""Solver steps after the transformer (CFG combine + UniPC / FlowMatch-Euler).

The oracle (oracle/solver.py) is pinned by what the mathematics fixes, since the
reference's schedulers live in diffusers (absent here) and its own tests stub
them: exactness on single-point flows, the measured order of accuracy on a
Gaussian data distribution whose flow ODE has a closed-form solution (UniPC-2 with
corrector: order 3; UniPC-1 with corrector: order 2; Euler: order 1), and planted
coefficient mistakes that must break those orders.  The host coefficient algebra
(ditserve_amd/solver.py) is checked against the oracle step by step; the HIP
kernel against the oracle in tests/test_gpu_solver.py.  The choice B(h) = expm1(-h)
("bh2", the Wan configuration) over B(h) = -h ("bh1") is not fixed by these
properties (both variants reach the same orders): that choice is parity unpinned."""
import math

import numpy as np
import pytest

from ditserve_amd import solver as ds
from oracle import solver as osv

MU, SD = 0.7, 0.4
Z = np.array([1.3, -0.6, 0.05, 2.1, -1.7])


def _vel(x, sig):
    """Exact flow velocity E[eps - x0 | x_sigma = x] for x0 ~ N(MU, SD^2)."""
    a = 1.0 - sig
    var = a * a * SD * SD + sig * sig
    d = x - a * MU
    return sig * d / var - (MU + a * SD * SD * d / var)


def _exact(sig):
    """The flow ODE solution through x(1) = Z."""
    a = 1.0 - sig
    return a * MU + math.sqrt(a * a * SD * SD + sig * sig) * Z


def _integrate(make, sigmas):
    o = make(sigmas)
    x = _exact(sigmas[0])
    for i in range(len(sigmas) - 1):
        x = o.step(_vel(x, sigmas[i]), x)
    return np.abs(x - _exact(sigmas[-1])).max()


def _ratios(make, ns=(32, 64, 128)):
    errs = [_integrate(make, np.linspace(0.9, 0.1, n + 1)) for n in ns]
    return [errs[i] / errs[i + 1] for i in range(len(errs) - 1)]


def test_unipc_order2_with_corrector_is_third_order():
    r = _ratios(lambda s: osv.UniPCFlowOracle(s, lower_order_final=False))
    assert min(r) > 6.0, r


def test_unipc_order1_with_corrector_is_second_order():
    r = _ratios(lambda s: osv.UniPCFlowOracle(s, solver_order=1, lower_order_final=False))
    assert all(3.3 < x < 4.5 for x in r), r


def test_unipc_without_corrector_is_second_order():
    r = _ratios(lambda s: osv.UniPCFlowOracle(s, disable_corrector=range(1000), lower_order_final=False))
    assert all(3.3 < x < 4.6 for x in r), r


def test_euler_is_first_order():
    r = _ratios(osv.FlowMatchEulerOracle)
    assert all(1.8 < x < 2.2 for x in r), r


@pytest.mark.parametrize("mistake", ["predictor_d1_sign", "corrector_rho_swap", "corrector_ignores_new_output"])
def test_planted_mistakes_break_the_order(monkeypatch, mistake):
    """A mistake planted in the oracle on the CPU must fail the order check."""
    if mistake == "predictor_d1_sign":
        orig = osv.UniPCFlowOracle._predict

        def bad(self, x, order):
            out = orig(self, x, order)
            if order == 2:  # flip the sign of the D1 term: subtract it twice
                out = 2 * orig(self, x, 1) - out
            return out
        monkeypatch.setattr(osv.UniPCFlowOracle, "_predict", bad)
    elif mistake == "corrector_rho_swap":
        orig_solve = np.linalg.solve
        monkeypatch.setattr(osv.np.linalg, "solve", lambda a, b: orig_solve(a, b)[::-1])
    else:
        orig_c = osv.UniPCFlowOracle._correct
        monkeypatch.setattr(osv.UniPCFlowOracle, "_correct",
                            lambda self, m, last, this, order: orig_c(self, self.model_outputs[-1], last, this, order))
    r = _ratios(lambda s: osv.UniPCFlowOracle(s, lower_order_final=False))
    assert min(r) < 6.0, r


def test_single_point_flows_are_exact():
    """With the exact velocity of one data point every data-prediction step lands
    on (1 - sigma) x0 + sigma eps: pins the x and m0 coefficients and the sign of h."""
    x0, eps = np.array([0.3, -1.2, 2.0]), np.array([0.9, 0.1, -0.4])
    for sig, make in ((osv.unipc_flow_sigmas(12, 3.0)[0], osv.UniPCFlowOracle),
                      (osv.flowmatch_sigmas(12, 3.0)[0], osv.FlowMatchEulerOracle)):
        o = make(sig)
        x = (1 - sig[0]) * x0 + sig[0] * eps
        for i in range(12):
            x = o.step(eps - x0, x)
            np.testing.assert_allclose(x, (1 - sig[i + 1]) * x0 + sig[i + 1] * eps, atol=1e-12)
        np.testing.assert_allclose(x, x0, atol=1e-12)


def test_sigma_tables():
    sig, ts = osv.unipc_flow_sigmas(50, 3.0)
    assert len(sig) == 51 and len(ts) == 50 and sig[-1] == 0.0
    assert np.all(np.diff(sig) < 0) and 0.999 < sig[0] < 1.0
    np.testing.assert_allclose(sig[1], osv.shift_sigmas(1.0 - (1.0 - 48 * 0.999 / 50 - 0.999 / 50), 3.0), rtol=1e-6)
    assert ts.dtype == np.int64 and ts[0] == 999
    fs, _ = osv.flowmatch_sigmas(28, 3.0)
    assert fs[0] == 1.0 and fs[-1] == 0.0 and np.all(np.diff(fs) < 0) and len(fs) == 29
    # shift 1 leaves the linspace untouched
    f1, _ = osv.flowmatch_sigmas(10, 1.0)
    np.testing.assert_allclose(f1[:-1], np.linspace(1.0, 0.001, 10), rtol=1e-6)
    np.testing.assert_allclose(osv.shift_sigmas([0.0, 0.5, 1.0], 3.0), [0.0, 0.75, 1.0])


def test_calculate_shift():
    """Endpoints of the linear rule and the reference's own ordering check
    (tests/python/test_domain_block_executor.py:698)."""
    assert math.isclose(ds.calculate_shift(256), 0.5) and math.isclose(ds.calculate_shift(4096), 1.15)
    assert ds.calculate_shift(1024) < ds.calculate_shift(2304) < ds.calculate_shift(4096)
    assert ds.calculate_shift(1024) == osv.calculate_shift(1024)


def _emulate(coef, x, c, u, xl, mp, mp2):
    """The kernel's per-element formula in float64."""
    g, sigma, ax, a0, a1, a2, a3, b0, b1, b2, bv = coef
    v = c if u is None else u + g * (c - u)
    m = x - sigma * v
    z = np.zeros_like(x)
    xc = ax * x + a0 * (z if xl is None else xl) + a1 * (z if mp is None else mp) + a2 * (z if mp2 is None else mp2) + a3 * m
    return b0 * xc + b1 * m + b2 * (z if mp is None else mp) + bv * v, xc, m


@pytest.mark.parametrize("steps,order", [(10, 2), (7, 1), (3, 2)])
def test_unipc_host_coefficients_match_oracle(steps, order):
    rng = np.random.default_rng(steps)
    sched = ds.UniPCFlowScheduler(flow_shift=3.0, solver_order=order)
    sched.set_timesteps(steps)
    sig, ts = osv.unipc_flow_sigmas(steps, 3.0)
    np.testing.assert_array_equal(sched.sigmas, sig)
    np.testing.assert_array_equal(sched.timesteps.numpy(), ts)
    ref = osv.UniPCFlowOracle(sig, solver_order=order)
    x = rng.standard_normal(64)
    xr = x.copy()
    xl = mp = mp2 = None
    for _ in range(steps):
        c, u = rng.standard_normal(64), rng.standard_normal(64)
        coef = sched.step_coefficients()
        coef[0] = 4.5
        xn, xc, m = _emulate(coef, x, c, u, xl, mp, mp2)
        xr = ref.step(osv.cfg(c, u, 4.5), xr)
        np.testing.assert_allclose(xn, xr, rtol=1e-10, atol=1e-12)
        x, xl, mp2, mp = xn, xc, mp, m


def test_flowmatch_host_sigmas_match_oracle():
    sched = ds.FlowMatchEulerScheduler(shift=3.0)
    sched.set_timesteps(28)
    sig, ts = osv.flowmatch_sigmas(28, 3.0)
    np.testing.assert_array_equal(sched.sigmas, sig)
    np.testing.assert_array_equal(sched.timesteps.numpy(), ts)
    dyn = ds.FlowMatchEulerScheduler(use_dynamic_shifting=True)
    mu = ds.calculate_shift(4096)
    dyn.set_timesteps(28, mu=mu)
    np.testing.assert_array_equal(dyn.sigmas, osv.flowmatch_sigmas(28, 3.0, mu=mu)[0])
