"""Oracle: the per-request solver steps that follow the transformer, in float64 numpy.

Test infrastructure only (see oracle/__init__.py).  The reference calls these
through diffusers' schedulers (diffusers 0.36.0, not vendored in the reference):
  Wan   - UniPCMultistepScheduler.step            workers/ditserve/models/wan/block.py:482-483,
          configured as the Wan pipelines ship it: prediction_type flow_prediction,
          use_flow_sigmas, flow_shift, solver_order 2, solver_type bh2, predict_x0,
          lower_order_final, final_sigmas_type zero, no external predictor
          (checks in workers/ditserve/models/wan/runtime.py:301-311,397-402;
          workers/ditserve/models/wan/parallel.py:738)
  SD3.5 - FlowMatchEulerDiscreteScheduler.step    workers/ditserve/models/sd35.py:952,
          timesteps from set_timesteps(steps, mu) workers/ditserve/models/sd35.py:837-862,
          dynamic shift mu from calculate_shift    workers/ditserve/models/sd35_batch.py:122-132
  CFG   - u + g * (c - u)                          workers/ditserve/models/wan/block.py:471,
                                                   workers/ditserve/models/sd35.py:949
The UniPC update is the published UniPC predictor/corrector (Zhao et al., 2023,
"UniPC: A Unified Predictor-Corrector Framework for Fast Sampling of Diffusion
Models"), data-prediction form with B(h) = expm1(-h) ("bh2"), on the flow
parameterisation alpha = 1 - sigma.  Pinning: exactness on single-point flows and
the measured order of accuracy on a Gaussian data distribution whose flow ODE has
a closed-form solution (tests/test_solver.py).  Equality with diffusers' own code
is not checked here (diffusers is absent): parity unpinned beyond those properties.
"""
import math

import numpy as np


def shift_sigmas(sigmas, shift):
    """The resolution shift of flow-matching schedules: s -> shift*s / (1 + (shift-1)*s)."""
    sigmas = np.asarray(sigmas, dtype=np.float64)
    return shift * sigmas / (1.0 + (shift - 1.0) * sigmas)


def calculate_shift(image_seq_len, base_seq_len=256, max_seq_len=4096, base_shift=0.5, max_shift=1.15):
    """workers/ditserve/models/sd35_batch.py:122-132."""
    m = (max_shift - base_shift) / max(1, (max_seq_len - base_seq_len))
    b = base_shift - m * base_seq_len
    return float(image_seq_len * m + b)


def time_shift_exp(mu, sigmas):
    """Dynamic (exponential) shift: e^mu / (e^mu + (1/s - 1))."""
    sigmas = np.asarray(sigmas, dtype=np.float64)
    return math.exp(mu) / (math.exp(mu) + (1.0 / sigmas - 1.0))


def unipc_flow_sigmas(steps, flow_shift, num_train_timesteps=1000):
    """UniPC with flow sigmas: `steps` descending sigmas from the shifted
    linspace(0, 1 - 1/N_train, steps + 1) without its 0 end, then a final 0; the
    model timesteps are sigma * N_train truncated to integers."""
    alphas = np.linspace(1.0, 1.0 / num_train_timesteps, steps + 1)
    sig = np.flip(shift_sigmas(1.0 - alphas, flow_shift))[:-1].copy()
    timesteps = (sig * num_train_timesteps).astype(np.float32).astype(np.int64)
    sigmas = np.concatenate([sig, [0.0]]).astype(np.float32).astype(np.float64)
    return sigmas, timesteps


def flowmatch_sigmas(steps, shift=3.0, num_train_timesteps=1000, mu=None):
    """FlowMatch-Euler: linspace between the (shifted) training sigma range,
    shifted again (static shift) or by exp(mu) (dynamic shift), then a final 0."""
    train = np.linspace(1.0, num_train_timesteps, num_train_timesteps)[::-1] / num_train_timesteps
    train = shift_sigmas(train, shift) if mu is None else train
    s_max, s_min = train[0], train[-1]
    t = np.linspace(s_max * num_train_timesteps, s_min * num_train_timesteps, steps)
    sig = t / num_train_timesteps
    sig = shift_sigmas(sig, shift) if mu is None else time_shift_exp(mu, sig)
    timesteps = (sig * num_train_timesteps).astype(np.float32)
    sigmas = np.concatenate([sig, [0.0]]).astype(np.float32).astype(np.float64)
    return sigmas, timesteps


def cfg(cond, uncond, guidance):
    """CFG combine, or the conditional output alone when there is no uncond branch."""
    if uncond is None:
        return np.asarray(cond, dtype=np.float64)
    return uncond + guidance * (cond - uncond)


class UniPCFlowOracle:
    """State and step of a UniPC (order 2, bh2, data prediction) flow sampler."""

    def __init__(self, sigmas, solver_order=2, disable_corrector=(), lower_order_final=True):
        self.sigmas = np.asarray(sigmas, dtype=np.float64)
        self.order = solver_order
        self.disable_corrector = set(disable_corrector)
        self.lower_order_final = lower_order_final
        self.model_outputs = [None] * solver_order
        self.lower_order_nums = 0
        self.this_order = 1
        self.last_sample = None
        self.step_index = 0

    @staticmethod
    def _lam(s):
        # lambda = log(alpha) - log(sigma), alpha = 1 - sigma; sigma = 0 gives +inf
        with np.errstate(divide="ignore"):
            return math.log(1.0 - s) - math.log(s) if s > 0 else math.inf

    def _phis(self, h):
        hh = -h
        h_phi_1 = math.expm1(hh)
        b_h = math.expm1(hh)
        return hh, h_phi_1, b_h

    def _rhs(self, hh, b_h, order):
        # b_k = h_phi_k * k! / B(h), h_phi_1 = expm1(hh)/hh - 1, h_phi_{k+1} = h_phi_k/hh - 1/(k+1)!
        h_phi_k = math.expm1(hh) / hh - 1.0
        fact = 1.0
        b = []
        for k in range(1, order + 1):
            b.append(h_phi_k * fact / b_h)
            fact *= k + 1
            h_phi_k = h_phi_k / hh - 1.0 / fact
        return b

    def _predict(self, x, order):
        """Predictor from sigma[i] to sigma[i+1] with m0 = model_outputs[-1]."""
        i = self.step_index
        s0, st = self.sigmas[i], self.sigmas[i + 1]
        m0 = self.model_outputs[-1]
        h = self._lam(st) - self._lam(s0)
        hh, h_phi_1, b_h = self._phis(h)
        alpha_t = 1.0 - st
        x_t_ = (st / s0) * x - alpha_t * h_phi_1 * m0
        if order == 2:
            m1 = self.model_outputs[-2]
            r1 = (self._lam(self.sigmas[i - 1]) - self._lam(s0)) / h
            d1 = (m1 - m0) / r1
            return x_t_ - alpha_t * b_h * 0.5 * d1
        return x_t_

    def _correct(self, this_m, last_sample, this_sample, order):
        """Corrector of the sample at sigma[i] with the new model output this_m."""
        i = self.step_index
        st, s0 = self.sigmas[i], self.sigmas[i - 1]
        m0 = self.model_outputs[-1]
        h = self._lam(st) - self._lam(s0)
        hh, h_phi_1, b_h = self._phis(h)
        alpha_t = 1.0 - st
        x_t_ = (st / s0) * last_sample - alpha_t * h_phi_1 * m0
        d1_t = this_m - m0
        if order == 1:
            return x_t_ - alpha_t * b_h * 0.5 * d1_t
        m1 = self.model_outputs[-2]
        r1 = (self._lam(self.sigmas[i - 2]) - self._lam(s0)) / h
        d1 = (m1 - m0) / r1
        rhs = self._rhs(hh, b_h, 2)
        rhos = np.linalg.solve(np.array([[1.0, 1.0], [r1, 1.0]]), np.array(rhs))
        return x_t_ - alpha_t * b_h * (rhos[0] * d1 + rhos[1] * d1_t)

    def step(self, velocity, sample):
        """One step with the (CFG-combined) velocity at sigma[step_index]."""
        x = np.asarray(sample, dtype=np.float64)
        m = x - self.sigmas[self.step_index] * np.asarray(velocity, dtype=np.float64)
        use_corrector = (self.step_index > 0 and (self.step_index - 1) not in self.disable_corrector
                         and self.last_sample is not None)
        if use_corrector:
            x = self._correct(m, self.last_sample, x, self.this_order)
        self.model_outputs = self.model_outputs[1:] + [m]
        n = len(self.sigmas) - 1
        this_order = min(self.order, n - self.step_index) if self.lower_order_final else self.order
        self.this_order = min(this_order, self.lower_order_nums + 1)
        self.last_sample = x
        prev = self._predict(x, self.this_order)
        if self.lower_order_nums < self.order:
            self.lower_order_nums += 1
        self.step_index += 1
        return prev


class FlowMatchEulerOracle:
    """FlowMatch-Euler: x_next = x + (sigma_next - sigma) * v."""

    def __init__(self, sigmas):
        self.sigmas = np.asarray(sigmas, dtype=np.float64)
        self.step_index = 0

    def step(self, velocity, sample):
        i = self.step_index
        out = np.asarray(sample, dtype=np.float64) + (self.sigmas[i + 1] - self.sigmas[i]) * np.asarray(velocity)
        self.step_index += 1
        return out
