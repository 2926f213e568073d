"""The Wan engine a worker's block executor drives, on the ditk kernels.

Same surface as the reference's xDiT engine (workers/ditserve/models/xdit/wan.py:35-122):
``begin_packet(state, branch)``, ``forward_block(packet, index)``,
``prediction(packet)``, ``forward(state, branch)``, ``activate(state, layout)``,
``attach_groups(groups)``, ``info()``, ``close()`` and the ``model`` / ``revision``
properties.  ``state`` is the worker's request state: ``latents``
[B, C, F, H, W], ``prompt_embeds`` / ``negative_prompt_embeds`` [B, L, text_dim],
``scheduler.timesteps`` and ``step_index`` (workers/ditserve/models/wan/runtime.py).
The executor calls these in the order of block.py:193-235 (begin) and
block.py:450-485 (blocks, then prediction of each branch, CFG combine and the
scheduler step).

Every call launches on the caller's current stream and allocates only through
the stream-aware caching allocator; packets carry ``record_stream`` on every
device object they hold.  So the reference's interleaved mode -- the uncond
branch's blocks on a side stream (block.py:237-300) -- gives the same results as
sequential execution when it sends ditk packets through its generic
``_forward_block`` path (block.py:254-266), i.e. ``engine.forward_block``: its
sublayer path would run the diffusers block's own modules on the packet, whose
layout (token-major ``[T, D]`` hidden rows, angle-table rotary) is ditk's.  One
GPU: a layout or group of more than one rank is rejected.
"""
import torch

from . import _lib
from .wan import WanTransformer


class DitkWanEngine:
    """Wan packet engine over a device-resident ``WanTransformer``.

    ``expand_timesteps``: Wan2.2 TI2V conditions every patch token on its own
    timestep (runtime.py:153-163); the ditk model takes them per request (all
    equal under the text-to-video mask)."""

    name = "ditk"

    def __init__(self, model, *, expand_timesteps=False, pipeline="WanPipeline"):
        if not isinstance(model, WanTransformer):
            raise ValueError("DitkWanEngine drives a ditserve_amd.wan.WanTransformer")
        self._model = model
        self.expand_timesteps = bool(expand_timesteps)
        self.pipeline = pipeline
        self._layout = None
        self._closed = False

    @property
    def model(self):
        return self._model

    @property
    def revision(self):
        return f"ditk-{int(_lib.load().ditk_version())}"

    # ------------------------------------------------------------ layout
    @staticmethod
    def _ranks(obj):
        for attr in ("ranks", "current_ranks"):
            if hasattr(obj, attr):
                return tuple(getattr(obj, attr))
        if isinstance(obj, (list, tuple)):
            return tuple(obj)
        return None

    def attach_groups(self, groups):
        """Rank groups of a sequence-parallel pool; only a single rank is served."""
        ranks = self._ranks(groups) if groups is not None else None
        if ranks is not None and len(ranks) > 1:
            raise ValueError("the ditk engine runs on one GPU: no sequence- or CFG-parallel groups")
        self._layout = None

    def activate(self, state, layout=None):
        """Check the request against the model and the layout (one rank, no CFG
        split) before any packet is built; returns the layout."""
        if self._closed:
            raise RuntimeError("engine is closed")
        if layout is not None:
            degree = getattr(layout, "degree", 1)
            cfg = getattr(layout, "cfg", 1)
            ranks = self._ranks(layout)
            if degree != 1 or cfg != 1 or (ranks is not None and len(ranks) != 1):
                raise ValueError("the ditk engine runs on one GPU: layout must have one rank and cfg 1")
        lat = state.latents
        if lat.dim() != 5 or lat.shape[1] != self._model.cfg.in_ch:
            raise ValueError(f"latents must be [B, {self._model.cfg.in_ch}, F, H, W], got {tuple(lat.shape)}")
        self._model._grid(lat.shape)
        self._layout = layout
        return layout

    # ------------------------------------------------------------ packets
    def _timestep(self, state):
        """workers/ditserve/models/wan/runtime.py:153-163: [B] (Wan2.1) or
        [B, F*(H/2)*(W/2)] (Wan2.2 TI2V), every token at the step's timestep."""
        lat = state.latents
        t = state.scheduler.timesteps[state.step_index]
        t = torch.as_tensor(t, dtype=torch.float32).reshape(())
        b = lat.shape[0]
        if not self.expand_timesteps:
            return t.expand(b).clone()
        f, h, w = lat.shape[2:]
        return t.expand(b, f * (h // 2) * (w // 2)).clone()

    def begin_packet(self, state, branch):
        self.activate(state, self._layout)
        if branch not in ("cond", "uncond"):
            raise ValueError("branch must be 'cond' or 'uncond'")
        encoder = state.prompt_embeds if branch == "cond" else state.negative_prompt_embeds
        return self._model.begin_packet(state.latents, self._timestep(state), encoder)

    def forward_block(self, packet, index):
        return self._model.forward_block(packet, index)

    def prediction(self, packet):
        return self._model.prediction(packet)

    def forward(self, state, branch):
        """begin_packet + every block + prediction (the whole-step path,
        runtime.py:686-700)."""
        packet = self.begin_packet(state, branch)
        for i in range(self._model.cfg.layers):
            self.forward_block(packet, i)
        return self.prediction(packet)

    def info(self):
        return dict(name=self.name, revision=self.revision, attention="ditk_flash_varlen", sp_ranks=[0],
                    pipeline=self.pipeline, transformer=type(self._model).__name__)

    def close(self):
        self._closed = True
