"""Per-request solver steps after the transformer: fused CFG combine + UniPC
(Wan) or FlowMatch-Euler (SD3.5), on the ditk_solver_step HIP kernel.

The reference drives diffusers' schedulers with
    latents = scheduler.step(prediction, t, latents, return_dict=False)[0]
(workers/ditserve/models/wan/block.py:482-483, workers/ditserve/models/wan/runtime.py:701,
workers/ditserve/models/sd35.py:952), after a separate CFG combine u + g (c - u)
(block.py:471, sd35.py:949).  These classes keep that surface —
``set_timesteps(steps)``, ``timesteps``, ``sigmas``, ``step(model_output, timestep,
sample, return_dict=False)`` — and ``step`` also takes ``uncond`` and ``guidance``
so that the CFG combine runs in the same kernel as the update.

Each step is a per-element linear combination of the sample, the model
outputs and two history buffers; its scalar coefficients are computed here in
float64 from the sigma table (host only, no device synchronisation):
  v  = uncond + g (cond - uncond)              (or cond)
  m  = x - sigma_i v                           data prediction of the flow model
  xc = corrector(x_last, m_prev, m_prev2, m)   (or x)
  x' = predictor(xc, m, m_prev)
UniPC follows the published predictor-corrector (Zhao et al., 2023) in its
data-prediction form with B(h) = expm1(-h), order 2 with a lower-order first
and final step, as diffusers' UniPCMultistepScheduler (flow_prediction,
use_flow_sigmas, solver_type bh2) is configured for Wan; the sigma tables are
the flow-shifted ones of those schedulers.
"""
import math

import numpy as np
import torch

from . import ops


def calculate_shift(image_seq_len, base_seq_len=256, max_seq_len=4096, base_shift=0.5, max_shift=1.15):
    """SD3 FlowMatch dynamic-resolution shift mu from the patch token count
    (workers/ditserve/models/sd35_batch.py:122-132): linear in the token count,
    base_shift at base_seq_len and max_shift at max_seq_len."""
    m = (max_shift - base_shift) / max(1, (max_seq_len - base_seq_len))
    return float(image_seq_len * m + base_shift - m * base_seq_len)


def _shift(s, shift):
    return shift * s / (1.0 + (shift - 1.0) * s)


def _lam(s):
    """log(alpha) - log(sigma) with alpha = 1 - sigma; +inf at sigma = 0."""
    return math.log(1.0 - s) - math.log(s) if s > 0 else math.inf


class _Base:
    num_train_timesteps = 1000

    def _alloc_like(self, sample):
        return torch.empty_like(sample, dtype=torch.float32)

    def _launch(self, coef, cond, sample, uncond, x_last=None, m_prev=None, m_prev2=None, x_corr=None, m_out=None):
        if sample.dtype != torch.float32 or cond.dtype != torch.float32:
            raise ValueError("solver steps run on fp32 latents and model outputs")
        return ops.solver_step(sample.contiguous(), cond.contiguous(), coef,
                               uncond=None if uncond is None else uncond.contiguous(), x_last=x_last,
                               m_prev=m_prev, m_prev2=m_prev2, x_corr=x_corr, m_out=m_out)


class UniPCFlowScheduler(_Base):
    """UniPC multistep sampler on flow sigmas (Wan's scheduler recipe)."""

    def __init__(self, flow_shift=3.0, solver_order=2, disable_corrector=(), lower_order_final=True,
                 num_train_timesteps=1000):
        if solver_order not in (1, 2):
            raise ValueError("solver_order must be 1 or 2")
        self.flow_shift = float(flow_shift)
        self.solver_order = solver_order
        self.disable_corrector = set(disable_corrector)
        self.lower_order_final = lower_order_final
        self.num_train_timesteps = num_train_timesteps
        self.sigmas = None
        self.timesteps = None

    def set_timesteps(self, num_inference_steps, device=None):
        n = int(num_inference_steps)
        alphas = np.linspace(1.0, 1.0 / self.num_train_timesteps, n + 1)
        sig = np.flip(_shift(1.0 - alphas, self.flow_shift))[:-1].copy()
        self.timesteps = torch.from_numpy((sig * self.num_train_timesteps).astype(np.float32).astype(np.int64))
        self.sigmas = np.concatenate([sig, [0.0]]).astype(np.float32).astype(np.float64)
        self.step_index = 0
        self.lower_order_nums = 0
        self.this_order = 1
        self._x_last = None
        self._m = [None, None]  # m_prev2, m_prev

    # coefficient algebra -------------------------------------------------------
    def _corrector(self, i, order):
        """x_c = a0 x_last + a1 m_prev + a2 m_prev2 + a3 m."""
        st, s0 = self.sigmas[i], self.sigmas[i - 1]
        h = _lam(st) - _lam(s0)
        hh = -h
        h_phi_1 = b_h = math.expm1(hh)
        alpha_t = 1.0 - st
        a0 = st / s0
        if order == 1:
            rho_t = 0.5
            return a0, -alpha_t * h_phi_1 + alpha_t * b_h * rho_t, 0.0, -alpha_t * b_h * rho_t
        r1 = (_lam(self.sigmas[i - 2]) - _lam(s0)) / h
        h_phi_k = math.expm1(hh) / hh - 1.0
        b = [h_phi_k / b_h, (h_phi_k / hh - 0.5) * 2.0 / b_h]
        det = 1.0 - r1  # R = [[1, 1], [r1, 1]]
        rho0 = (b[0] - b[1]) / det
        rho1 = (b[1] - r1 * b[0]) / det
        a1 = -alpha_t * h_phi_1 + alpha_t * b_h * (rho0 / r1 + rho1)
        a2 = -alpha_t * b_h * rho0 / r1
        a3 = -alpha_t * b_h * rho1
        return a0, a1, a2, a3

    def _predictor(self, i, order):
        """x' = b0 x_c + b1 m + b2 m_prev."""
        s0, st = self.sigmas[i], self.sigmas[i + 1]
        h = _lam(st) - _lam(s0)
        hh = -h
        h_phi_1 = b_h = math.expm1(hh)
        alpha_t = 1.0 - st
        b0 = st / s0
        if order == 1:
            return b0, -alpha_t * h_phi_1, 0.0
        r1 = (_lam(self.sigmas[i - 1]) - _lam(s0)) / h
        return b0, -alpha_t * h_phi_1 + 0.5 * alpha_t * b_h / r1, -0.5 * alpha_t * b_h / r1

    def step_coefficients(self):
        """The 11 kernel coefficients (without g) of the current step, and the
        history it reads; advances the scheduler state."""
        i = self.step_index
        use_corrector = i > 0 and (i - 1) not in self.disable_corrector  # every step leaves a last sample
        if use_corrector:
            ax, (a0, a1, a2, a3) = 0.0, self._corrector(i, self.this_order)
        else:
            ax, a0, a1, a2, a3 = 1.0, 0.0, 0.0, 0.0, 0.0
        n = len(self.sigmas) - 1
        order = min(self.solver_order, n - i) if self.lower_order_final else self.solver_order
        order = min(order, self.lower_order_nums + 1)
        b0, b1, b2 = self._predictor(i, order)
        coef = [0.0, float(self.sigmas[i]), ax, a0, a1, a2, a3, b0, b1, b2, 0.0]
        self.this_order = order
        if self.lower_order_nums < self.solver_order:
            self.lower_order_nums += 1
        self.step_index += 1
        return coef

    def step(self, model_output, timestep, sample, return_dict=False, uncond=None, guidance=1.0):
        """x_{i+1} from x_i and the model output at timesteps[step_index] (the
        conditional one, combined with ``uncond`` by ``guidance`` when given)."""
        if self.sigmas is None:
            raise RuntimeError("call set_timesteps first")
        if self.step_index >= len(self.timesteps):
            raise RuntimeError("no steps left")
        m_prev2, m_prev = self._m
        coef = self.step_coefficients()
        coef[0] = float(guidance)
        x_corr = self._x_last if self._x_last is not None else self._alloc_like(sample)
        m_out = m_prev2 if m_prev2 is not None else self._alloc_like(sample)
        out = self._launch(coef, model_output, sample, uncond, x_last=self._x_last, m_prev=m_prev,
                           m_prev2=m_prev2, x_corr=x_corr, m_out=m_out)
        self._x_last = x_corr
        self._m = [m_prev, m_out]
        return (out,)


class FlowMatchEulerScheduler(_Base):
    """FlowMatch-Euler sampler (SD3.5's scheduler recipe): x' = x + (s' - s) v."""

    def __init__(self, shift=3.0, use_dynamic_shifting=False, num_train_timesteps=1000):
        self.shift = float(shift)
        self.use_dynamic_shifting = use_dynamic_shifting
        self.num_train_timesteps = num_train_timesteps
        self.sigmas = None
        self.timesteps = None

    def set_timesteps(self, num_inference_steps, device=None, mu=None):
        n = int(num_inference_steps)
        nt = self.num_train_timesteps
        train = np.linspace(1.0, nt, nt)[::-1] / nt
        if not self.use_dynamic_shifting:
            train = _shift(train, self.shift)
        t = np.linspace(train[0] * nt, train[-1] * nt, n)
        sig = t / nt
        if self.use_dynamic_shifting:
            if mu is None:
                raise ValueError("dynamic shifting needs mu")
            sig = math.exp(mu) / (math.exp(mu) + (1.0 / sig - 1.0))
        else:
            sig = _shift(sig, self.shift)
        self.timesteps = torch.from_numpy((sig * nt).astype(np.float32))
        self.sigmas = np.concatenate([sig, [0.0]]).astype(np.float32).astype(np.float64)
        self.step_index = 0

    def step(self, model_output, timestep, sample, return_dict=False, uncond=None, guidance=1.0):
        if self.sigmas is None:
            raise RuntimeError("call set_timesteps first")
        i = self.step_index
        if i >= len(self.timesteps):
            raise RuntimeError("no steps left")
        coef = [float(guidance), float(self.sigmas[i]), 1.0, 0.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0,
                float(self.sigmas[i + 1] - self.sigmas[i])]
        self.step_index += 1
        return (self._launch(coef, model_output, sample, uncond),)
