"""Packed block executor: the worker's block-quantum protocol over step-level
packed requests.

The reference's executor (workers/ditserve/models/wan/block.py:83-620) advances
one request by a quantum of transformer blocks, commits the solver step when the
last block finishes, and reports each quantum to the controller as a row
(block.py:405-412):
  kind="block_quantum", step_index, start_block, next_block, blocks,
  step_completed, ms, block_cuda_ms=[{branch, block, ms}], ...
plus a per-request ``step`` event at every commit (block.py:489-491).  Here one
packet holds every member request's conditional and unconditional branch as
segments of one varlen token batch, so a quantum advances all of them at once
(branch "packed"); the commit runs the prediction epilogue, then the fused CFG
combine + UniPC update per request (ditserve_amd.solver).  Quanta may stop at
any block boundary; ``export`` / ``load`` carry a mid-step executor through the
block-packet wire format (ditserve_amd.packet).  All work launches on the
caller's current stream; every call returns after its GPU work has completed,
as the reference's quanta do.
"""
import time

import torch

from . import packet as wire
from .packing import token_packing_stats
from .solver import UniPCFlowScheduler


class Request:
    """One generation request: latent, text contexts, guidance and its own solver."""

    def __init__(self, latents, prompt_embeds, negative_prompt_embeds=None, guidance_scale=5.0, steps=50,
                 flow_shift=3.0, request_id=None):
        if latents.dim() != 4:
            raise ValueError("latents must be [C, F, H, W]")
        self.latents = latents.float().contiguous()
        self.prompt_embeds = prompt_embeds
        self.negative_prompt_embeds = negative_prompt_embeds
        self.guidance_scale = float(guidance_scale)
        self.cfg = negative_prompt_embeds is not None and self.guidance_scale > 1.0
        self.scheduler = UniPCFlowScheduler(flow_shift=flow_shift)
        self.scheduler.set_timesteps(steps)
        self.steps = int(steps)
        self.request_id = request_id
        self.events = []

    @property
    def step_index(self):
        return self.scheduler.step_index

    @property
    def finished(self):
        return self.step_index >= self.steps


class PackedBlockExecutor:
    """Advances a set of requests through packed solver steps in block quanta."""

    def __init__(self, model):
        self.model = model
        self.requests = None
        self.packet = None
        self.next_block = 0
        self._advancing = False

    def _segments(self):
        """(request, branch) of every packet segment, in packet order."""
        out = []
        for r in self.requests:
            out.append((r, "cond"))
            if r.cfg:
                out.append((r, "uncond"))
        return out

    def _begin(self):
        lats, ts, texts = [], [], []
        for r, branch in self._segments():
            lats.append(r.latents)
            ts.append(float(r.scheduler.timesteps[r.step_index]))
            texts.append(r.prompt_embeds if branch == "cond" else r.negative_prompt_embeds)
        self.packet = self.model.begin_packed_packet(lats, ts, texts)
        self.next_block = 0

    def _commit(self):
        outs = self.model.prediction_packed(self.packet)
        j = 0
        for r in self.requests:
            cond = outs[j]
            uncond = outs[j + 1] if r.cfg else None
            j += 2 if r.cfg else 1
            t = r.scheduler.timesteps[r.step_index]
            shape = r.latents.shape
            r.latents = r.scheduler.step(cond.reshape(shape), t, r.latents, uncond=None if uncond is None
                                         else uncond.reshape(shape), guidance=r.guidance_scale)[0]
            r.events.append(dict(kind="step", step_index=r.step_index - 1, completed_steps=r.step_index,
                                 path="compute", executor="packed_blocks"))
        self.packet = None
        self.next_block = 0

    def attach(self, requests):
        """Set the member requests; only between solver steps."""
        if self.packet is not None:
            raise ValueError("cannot change members inside a solver step")
        if not requests or any(r.finished for r in requests):
            raise ValueError("requests must be non-empty and have remaining steps")
        self.requests = list(requests)

    def advance(self, blocks=1, observe=False):
        """Run at most ``blocks`` blocks, stopping no later than one solver commit."""
        if type(blocks) is not int or blocks < 1:
            raise ValueError("blocks must be a positive integer")
        if self.requests is None:
            raise ValueError("attach requests first")
        if self._advancing:
            raise RuntimeError("overlapping block execution")
        self._advancing = True
        try:
            torch.cuda.synchronize()
            started = time.perf_counter()
            if self.packet is None:
                if any(r.finished for r in self.requests):
                    raise ValueError("a member request has no remaining steps")
                self._begin()
            steps = [r.step_index for r in self.requests]
            start_block, events, executed, completed = self.next_block, [], 0, False
            layers = self.model.cfg.layers
            while executed < blocks:
                if observe:
                    a, z = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record()
                self.model.forward_block(self.packet, self.next_block)
                if observe:
                    z.record()
                    events.append((self.next_block, a, z))
                executed += 1
                self.next_block += 1
                if self.next_block == layers:
                    self._commit()
                    completed = True
                    break
            torch.cuda.synchronize()
            pt, ph, pw = self.model.cfg.patch
            counts = [r.latents[0].numel() // (pt * ph * pw) for r, _ in self._segments()]
            return dict(kind="block_quantum", step_index=steps, branch="packed", start_block=start_block,
                        next_block=self.next_block, blocks=executed, step_completed=completed,
                        ms=(time.perf_counter() - started) * 1000.0,
                        block_cuda_ms=[dict(branch="packed", block=i, ms=float(a.elapsed_time(z)))
                                       for i, a, z in events],
                        request_ids=[r.request_id for r in self.requests],
                        sequence_packing=True, packing=token_packing_stats(counts))
        finally:
            self._advancing = False

    def step(self, observe=False):
        """The rest of the current solver step (or one whole step)."""
        return self.advance(self.model.cfg.layers - self.next_block if self.packet is not None
                            else self.model.cfg.layers, observe=observe)

    def export(self):
        """Wire payload of a mid-step executor: the block packet plus where the
        step stands; requests' solver state stays with the requests."""
        if self.packet is None:
            raise ValueError("nothing to export between solver steps")
        payload, stats = wire.export_packet(self.packet)
        payload["manifest"]["layout"].update(next_block=self.next_block,
                                             committed_steps=[r.step_index for r in self.requests])
        return payload, stats

    def load(self, payload, requests):
        """Resume a mid-step payload with the same member requests."""
        if self.packet is not None or self._advancing:
            raise ValueError("executor is busy")
        layout = payload["manifest"]["layout"]
        if [r.step_index for r in requests] != layout["committed_steps"]:
            raise ValueError("block packet and request solver steps disagree")
        self.requests = list(requests)
        self.packet = wire.import_packet(payload, self.model)
        self.next_block = int(layout["next_block"])
