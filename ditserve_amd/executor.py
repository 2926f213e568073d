"""Packed block executor: the worker's block-quantum protocol over step-level
packed requests.

The reference's executor (workers/ditserve/models/wan/block.py:83-627) advances
one request by a quantum of transformer blocks, commits the solver step when the
last block finishes, and reports each quantum to the controller as a row
(block.py:611-617):
  kind="block_quantum", step_index, branch, start_block, next_block, next_branch,
  blocks, step_completed, ms, doorbell_stop, released_cache_on_stop,
  block_cuda_ms=[{branch, block, ms}], extra_state_bytes
plus a per-request ``step`` event at every commit (block.py:489-491).  Here one
packet holds every member request's conditional and unconditional branch as
segments of one varlen token batch, so a quantum advances all of them at once
and returns one row per member request, as the reference's lockstep pair does
(``advance_pair``, block.py:701-838: ``paired=True``; here ``packed=True``).
The commit runs the prediction epilogue, then the fused CFG combine + UniPC
update per request (ditserve_amd.solver).

Quanta may stop at any block boundary, after ``blocks`` blocks or when the
controller's doorbell rings (checked every ``check_every`` blocks, with the host
kept within one check interval of the GPU, as block.py:497-509,629-690 does).
``export`` / ``import_state`` carry an executor through the block-packet wire
format at any block boundary, solver state included (block.py:885-1007).
``advance_batch`` runs whole solver steps and reports them in the result shape
of the reference's batched advance (workers/ditserve/models/sd35.py:1025-1164).
All work launches on the caller's current stream; every call returns after its
GPU work has completed, as the reference's quanta do.
"""
import hashlib
import json
import time

import numpy as np
import torch

from . import packet as wire
from .packing import token_packing_stats
from .solver import UniPCFlowScheduler

# The reference's block_quantum row (block.py:611-617) and the fields this executor adds.
QUANTUM_ROW_FIELDS = frozenset({
    "kind", "step_index", "branch", "start_block", "next_block", "next_branch", "blocks", "step_completed", "ms",
    "doorbell_stop", "released_cache_on_stop", "block_cuda_ms", "extra_state_bytes"})
PACKED_ROW_FIELDS = frozenset({"packed", "request_id", "sequence_packing", "packing"})
# The reference's batched-advance result (workers/ditserve/models/sd35.py:1148-1159).
BATCH_RESULT_FIELDS = frozenset({
    "results", "batch_size", "quantum", "model_ms", "attention", "bubble_free", "sequence_packing", "packing",
    "step_meta", "memory_after"})
BASE_SCHEMA = "ditk.packed-request-state.v1"
_SOLVER_SCALARS = ("flow_shift", "solver_order", "lower_order_final", "num_train_timesteps", "step_index",
                   "lower_order_nums", "this_order")


def progress(step, steps, *, done=None, next_action=None):
    """Progress record of a request (workers/ditserve/models/base.py:76-79)."""
    done = step >= steps if done is None else bool(done)
    return dict(step=step, steps=steps, done=done, next_action=next_action or ("finish" if done else "advance"))


def memory():
    """Device memory summary in the reference's form (sd35.py:149-155)."""
    if torch.cuda.is_available():
        return dict(allocated_mb=round(torch.cuda.memory_allocated() / (1 << 20), 2),
                    reserved_mb=round(torch.cuda.memory_reserved() / (1 << 20), 2))
    return dict(allocated_mb=0.0, reserved_mb=0.0)


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

    @property
    def branch(self):
        """Branches this request's packet segments carry."""
        return "cond+uncond" if self.cfg else "cond"

    # ------------------------------------------------------------ wire format
    def export_state(self, prefix):
        """(metadata, tensors) of the request and its UniPC state; tensor names under
        ``prefix``, solver tensors named as the reference's cache-off wire names them
        (solver.last_sample, solver.model_outputs.<i>, solver.sigmas, solver.timesteps;
        workers/ditserve/models/wan/parallel.py:765-775)."""
        s = self.scheduler
        tensors = {"latents": self.latents, "prompt_embeds": self.prompt_embeds,
                   "negative_prompt_embeds": self.negative_prompt_embeds,
                   "solver.last_sample": s._x_last, "solver.model_outputs.0": s._m[0],
                   "solver.model_outputs.1": s._m[1], "solver.sigmas": torch.from_numpy(np.asarray(s.sigmas)),
                   "solver.timesteps": s.timesteps}
        meta = dict(request_id=self.request_id, guidance_scale=self.guidance_scale, steps=self.steps,
                    step_index=self.step_index, cfg=self.cfg,
                    scheduler={**{k: getattr(s, k) for k in _SOLVER_SCALARS},
                               "disable_corrector": sorted(s.disable_corrector)},
                    references={k: (None if v is None else prefix + k) for k, v in tensors.items()},
                    devices={k: v.device.type for k, v in tensors.items() if v is not None})
        return meta, {prefix + k: v.detach().cpu().clone().contiguous() for k, v in tensors.items() if v is not None}

    @classmethod
    def import_state(cls, meta, tensors, device):
        refs = meta["references"]

        def get(name):
            key = refs[name]
            if key is None:
                return None
            t = tensors[key]
            return t.to(device) if meta["devices"].get(name) == "cuda" else t.clone()
        sc = meta["scheduler"]
        r = cls.__new__(cls)
        r.latents = get("latents")
        r.prompt_embeds = get("prompt_embeds")
        r.negative_prompt_embeds = get("negative_prompt_embeds")
        r.guidance_scale = float(meta["guidance_scale"])
        r.cfg = bool(meta["cfg"])
        r.steps = int(meta["steps"])
        r.request_id = meta["request_id"]
        r.events = []
        s = UniPCFlowScheduler(flow_shift=sc["flow_shift"], solver_order=sc["solver_order"],
                               disable_corrector=sc["disable_corrector"], lower_order_final=sc["lower_order_final"],
                               num_train_timesteps=sc["num_train_timesteps"])
        s.set_timesteps(r.steps)
        sig = get("solver.sigmas").double().numpy()
        if not np.array_equal(sig, s.sigmas) or not torch.equal(get("solver.timesteps").cpu(), s.timesteps):
            raise ValueError("request solver schedule does not match its configuration")
        s.step_index, s.lower_order_nums, s.this_order = sc["step_index"], sc["lower_order_nums"], sc["this_order"]
        s._x_last = get("solver.last_sample")
        s._m = [get("solver.model_outputs.0"), get("solver.model_outputs.1")]
        r.scheduler = s
        if r.step_index != int(meta["step_index"]):
            raise ValueError("request step index and solver state disagree")
        return r


def _canonical(obj):
    return json.dumps(obj, sort_keys=True, separators=(",", ":"))


def _unique_bytes(values):
    """Bytes of the distinct device storages reachable from ``values``."""
    seen, total = set(), 0

    def visit(v):
        nonlocal total
        if torch.is_tensor(v):
            st = v.untyped_storage()
            key = (str(v.device), st.data_ptr(), st.nbytes())
            if key not in seen:
                seen.add(key)
                total += st.nbytes()
        elif isinstance(v, dict):
            for x in v.values():
                visit(x)
        elif isinstance(v, (list, tuple)):
            for x in v:
                visit(x)
        elif hasattr(v, "device_tensors"):
            for x in v.device_tensors():
                visit(x)
    visit(values)
    return total


class PackedBlockExecutor:
    """Advances a set of requests through packed solver steps in block quanta.

    ``release_cache_on_stop``: return cached device memory to the driver when a
    quantum stops inside a step (block.py:601-608)."""

    def __init__(self, model, *, release_cache_on_stop=False):
        self.model = model
        self.requests = None
        self.packet = None
        self.next_block = 0
        self.release_cache_on_stop = bool(release_cache_on_stop)
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
                                 path="compute", executor="packed_blocks", cfg_folded=False))
        self.packet = None
        self.next_block = 0

    def _token_counts(self):
        pt, ph, pw = self.model.cfg.patch
        return [r.latents[0].numel() // (pt * ph * pw) for r, _ in self._segments()]

    def attach(self, requests):
        """Set the member requests; only between solver steps."""
        if self.packet is not None:
            raise ValueError("cannot change members inside a solver step")
        if not requests or any(r.finished for r in requests):
            raise ValueError("requests must be non-empty and have remaining steps")
        self.requests = list(requests)

    def extra_state_bytes(self):
        """Unique device storage the in-flight packet retains (shared by its members)."""
        return int(_unique_bytes(self.packet)) if self.packet is not None else 0

    def quantum(self, policy):
        """Blocks of one quantum under a preemption policy (block.py:871-882):
        "step" (a whole solver step: both CFG branches run inside the packet),
        "cfg" (the rest of the step) or "block-<n>"."""
        layers = self.model.cfg.layers
        if policy in ("step", "cfg"):
            return layers - self.next_block if (policy == "cfg" and self.packet is not None) else layers
        if policy.startswith("block-"):
            return int(policy.split("-", 1)[1])
        raise ValueError("unknown preemption policy: " + policy)

    def advance(self, blocks=1, *, observe=False, check_budget=lambda: None, doorbell=None, check_every=0):
        """Run at most ``blocks`` blocks, stopping no later than one solver commit,
        or earlier at a check point where ``doorbell()`` is true.  Returns one
        quantum row per member request."""
        if type(blocks) is not int or blocks < 1:
            raise ValueError("blocks must be a positive integer")
        if doorbell is not None and (type(check_every) is not int or check_every < 1):
            raise ValueError("check_every must be a positive integer with a doorbell")
        if self.requests is None:
            raise ValueError("attach requests first")
        if self._advancing:
            raise RuntimeError("overlapping/reentrant GPU block execution")
        if self.packet is None and any(r.finished for r in self.requests):
            raise ValueError("a member request has no remaining steps")
        check_budget()
        self._advancing = True
        try:
            torch.cuda.synchronize()
            started = time.perf_counter()
            steps = [r.step_index for r in self.requests]
            start_block, events, executed, completed = self.next_block, [], 0, False
            iterations, pending, rung = 0, [], False
            layers = self.model.cfg.layers
            while executed < blocks:
                check_budget()
                if self.packet is None:
                    self._begin()
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
                iterations += 1
                if doorbell is not None and executed < blocks and iterations % check_every == 0:
                    # keep the host at most one check interval ahead of the GPU
                    mark = torch.cuda.Event()
                    mark.record()
                    pending.append(mark)
                    if len(pending) > 1:
                        pending.pop(0).synchronize()
                    if doorbell():
                        rung = True
                        break
            extra = self.extra_state_bytes()
            torch.cuda.synchronize()
            released = bool(not completed and self.release_cache_on_stop)
            if released:
                torch.cuda.empty_cache()
            wall_ms = (time.perf_counter() - started) * 1000.0
            cuda_ms = [dict(branch="packed", block=i, ms=float(a.elapsed_time(z))) for i, a, z in events]
            packing = token_packing_stats(self._token_counts())
            rows = []
            for r, step in zip(self.requests, steps):
                row = dict(kind="block_quantum", step_index=step, branch=r.branch, start_block=start_block,
                           next_block=self.next_block, next_branch=r.branch, blocks=executed,
                           step_completed=completed, ms=wall_ms, doorbell_stop=rung, released_cache_on_stop=released,
                           block_cuda_ms=cuda_ms, extra_state_bytes=extra, packed=True, request_id=r.request_id,
                           sequence_packing=True, packing=packing)
                r.events.append(row)
                rows.append(row)
            return rows
        finally:
            self._advancing = False

    def step(self, observe=False):
        """The rest of the current solver step (or one whole step)."""
        return self.advance(self.quantum("cfg"), observe=observe)

    def advance_batch(self, steps=1, *, state_ids=None):
        """Whole solver steps of every member request (``steps`` each, fewer for
        requests that finish), reported as the reference's batched advance result
        (workers/ditserve/models/sd35.py:1097-1164): per-request progress, the wall
        time, the packing summary of the batch and the last step's packing meta."""
        if type(steps) is not int or steps < 1:
            raise ValueError("steps must be a positive integer")
        if self.packet is not None:
            raise ValueError("advance_batch runs whole solver steps: finish the open step first")
        if self.requests is None:
            raise ValueError("attach requests first")
        ids = state_ids if state_ids is not None else [r.request_id for r in self.requests]
        if len(ids) != len(self.requests):
            raise ValueError("one state id per member request")
        torch.cuda.synchronize()
        started = time.perf_counter()
        members = self.requests
        step_meta = {}
        try:
            for _ in range(steps):
                active = [r for r in members if not r.finished]
                if not active:
                    break
                self.requests = active
                cu = [0]
                for n in self._token_counts():
                    cu.append(cu[-1] + n)
                self.advance(self.model.cfg.layers)
                step_meta = {"sequence_packed": True, "attention_backend": "ditk_flash_varlen",
                             "attention_provider": "ditk", "packed_segments": len(cu) - 1,
                             "cu_seqlens_img": cu, "packed_image_tokens": cu[-1],
                             "padded_image_tokens": (len(cu) - 1) * max(b - a for a, b in zip(cu, cu[1:])),
                             "vector_timesteps": [float(r.scheduler.timesteps[r.step_index - 1]) for r in active]}
                step_meta["padding_saved_tokens"] = step_meta["padded_image_tokens"] - cu[-1]
        finally:
            self.requests = members
        torch.cuda.synchronize()
        elapsed_ms = (time.perf_counter() - started) * 1000.0
        results = [dict(state_id=sid, progress=progress(r.step_index, r.steps), paused=not r.finished)
                   for sid, r in zip(ids, members)]
        return dict(results=results, batch_size=len(members), quantum="continuous_batch",
                    model_ms=round(elapsed_ms, 3), attention="ditk", bubble_free=False,
                    sequence_packing=bool(step_meta.get("sequence_packed", False)),
                    packing=token_packing_stats(self._token_counts()), step_meta=step_meta, memory_after=memory())

    # ------------------------------------------------------------ wire format
    def export(self):
        """(payload, stats) of the executor at a block boundary: the block packet
        (when inside a step) and every member's request and solver state, in the
        reference's manifest layout (block.py:908-945): schema, base, layout with
        committed_step / branch / next_block / packet / conditional / folded, and per
        extra tensor its SHA-256 and strides."""
        if self._advancing:
            raise RuntimeError("cannot export during block execution")
        if self.requests is None:
            raise ValueError("nothing attached")
        torch.cuda.synchronize()
        started = time.perf_counter()
        metas, base_tensors = [], {}
        for i, r in enumerate(self.requests):
            meta, tens = r.export_state(f"request.{i}.")
            metas.append(meta)
            base_tensors.update(tens)
        base = dict(schema=BASE_SCHEMA, requests=metas,
                    tensor_hashes={k: wire.digest(v) for k, v in base_tensors.items()})
        base["state_sha256"] = hashlib.sha256(_canonical(dict(base)).encode()).hexdigest()
        layout = dict(committed_step=[r.step_index for r in self.requests], branch="packed",
                      next_block=self.next_block, packet=self.packet is not None, conditional=False, folded=False,
                      engine=wire.engine_info())
        tensors = dict(base_tensors)
        extra = {}
        if self.packet is not None:
            pkt_payload, _ = wire.export_packet(self.packet)
            layout.update({k: v for k, v in pkt_payload["manifest"]["layout"].items() if k != "packet"})
            extra = pkt_payload["tensors"]
            tensors.update(extra)
        manifest = dict(schema=wire.PACKET_SCHEMA, base=base, layout=layout,
                        packet_sha256={k: wire.digest(v) for k, v in extra.items()},
                        strides={k: list(v.stride()) for k, v in extra.items()})
        packet_bytes = sum(v.numel() * v.element_size() for v in extra.values())
        return dict(manifest=manifest, tensors=tensors), dict(
            export_ms=(time.perf_counter() - started) * 1000.0, packet_bytes=packet_bytes,
            transfer_bytes=sum(v.numel() * v.element_size() for v in tensors.values()))

    @classmethod
    def import_state(cls, payload, model, **kwargs):
        """Rebuild an exported executor on ``model``'s device (block.py:948-1007):
        verify the schema, the engine revision, every tensor checksum and stride and
        the base state checksum, then restore the requests, their solver state and
        the packet.  Returns the executor."""
        manifest, tensors = payload["manifest"], payload["tensors"]
        if manifest.get("schema") != wire.PACKET_SCHEMA:
            raise ValueError("unknown block packet schema")
        layout, base = manifest["layout"], manifest["base"]
        if layout.get("engine", {}).get("revision") != wire.engine_info()["revision"]:
            raise ValueError("block packet engine revision mismatch")
        if base.get("schema") != BASE_SCHEMA:
            raise ValueError("unknown request state schema")
        names = set(manifest["packet_sha256"])
        base_names = set(base["tensor_hashes"])
        if set(tensors) != base_names | names:
            raise ValueError("block packet tensor set mismatch")
        for name in names:
            if (wire.digest(tensors[name]) != manifest["packet_sha256"][name]
                    or list(tensors[name].stride()) != manifest["strides"][name]):
                raise ValueError("block packet tensor checksum or layout mismatch: " + name)
        for name in base_names:
            if wire.digest(tensors[name]) != base["tensor_hashes"][name]:
                raise ValueError("request state tensor checksum mismatch: " + name)
        check = {k: v for k, v in base.items() if k != "state_sha256"}
        if hashlib.sha256(_canonical(check).encode()).hexdigest() != base["state_sha256"]:
            raise ValueError("request state manifest checksum mismatch")
        requests = [Request.import_state(m, tensors, model.device) for m in base["requests"]]
        if [r.step_index for r in requests] != list(layout["committed_step"]):
            raise ValueError("block packet and request solver steps disagree")
        if layout["folded"] or layout["conditional"]:
            raise ValueError("CFG-folded or split-branch packets are not produced by this executor")
        ex = cls(model, **kwargs)
        ex.requests = requests
        ex.next_block = int(layout["next_block"])
        if layout["packet"]:
            pkt = dict(manifest=dict(schema=wire.PACKET_SCHEMA, layout=layout,
                                     packet_sha256=manifest["packet_sha256"], strides=manifest["strides"]),
                       tensors={k: tensors[k] for k in names})
            ex.packet = wire.import_packet(pkt, model)
        elif ex.next_block:
            raise ValueError("a block boundary inside a step needs its packet")
        return ex
