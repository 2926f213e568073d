"""Block-packet wire format: a packet exported at a block boundary inside a
solver step (preemption, migration) and rebuilt on another worker.

Follows the reference's codec (workers/ditserve/models/wan/block.py:12-19 schema
names and digest, :885-945 export, :948-1007 import): a manifest with the
schema, a layout of plain JSON values and, per tensor, its SHA-256 over the raw
bytes and its strides; the tensors themselves as dense CPU copies named
``packet.<name>`` and ``packet.rotary.<i>``.  The packet tensors of the ditk
engine are dense by construction:
  hidden     [T, D] bf16       packed token rows of all requests
  encoder    [R*L, D] bf16     text rows, L per request
  temb       [R, D] bf16
  projected  [R, 6, D] fp32
  rotary     two RoPE angle tables [max_pos, head_dim/2] fp32
and the layout carries the per-request grids (thw) and shapes from which the
segment tables are rebuilt (WanTransformer.resolve_packet).  Per-token RoPE
tensors are not carried: the kernel rotates from the tables and the grids.
"""
import hashlib

import torch

PACKET_SCHEMA = "ditserve.wan-block-packet.v2"  # the engine-backed schema of block.py:13
PACKET_TENSORS = ("hidden", "encoder", "temb", "projected")


def digest(t):
    """SHA-256 of a tensor's raw bytes (block.py:17-18)."""
    return hashlib.sha256(t.detach().cpu().contiguous().reshape(-1).view(torch.uint8).numpy().tobytes()).hexdigest()


def engine_info():
    """Engine name and revision, as the reference's engine_info() reports them
    (workers/ditserve/models/xdit/__init__.py:7-8); a payload imports only into an
    engine of the same revision."""
    from . import _lib
    return {"name": "ditk", "revision": f"ditk-{int(_lib.load().ditk_version())}"}


def export_packet(packet, engine=None):
    """(payload, stats): payload = {manifest, tensors} with CPU tensors."""
    extra = {f"packet.{name}": packet[name] for name in PACKET_TENSORS}
    for i, t in enumerate(packet["rotary"]):
        extra[f"packet.rotary.{i}"] = t
    tensors = {name: t.detach().cpu().clone() for name, t in extra.items()}
    layout = dict(packet=True, shape=[list(map(int, s)) for s in packet["shape"]], rotary=len(tuple(packet["rotary"])),
                  xdit={"pad_amount": int(packet["pad_amount"]), "local_rows": int(packet["local_rows"]),
                        "valid_kv_len": packet["valid_kv_len"],
                        "thw": [list(map(int, g)) for g in packet["thw"]]},
                  engine=engine if engine is not None else engine_info())
    if "text_lens" in packet:
        layout["text_lens"] = [int(x) for x in packet["text_lens"]]
    manifest = dict(schema=PACKET_SCHEMA, layout=layout,
                    packet_sha256={name: digest(t) for name, t in tensors.items()},
                    strides={name: list(t.stride()) for name, t in tensors.items()})
    nbytes = sum(t.numel() * t.element_size() for t in tensors.values())
    return dict(manifest=manifest, tensors=tensors), dict(packet_bytes=nbytes)


def import_packet(payload, model, engine=None):
    """Verify a payload and rebuild the packet on ``model``'s device."""
    manifest, tensors = payload["manifest"], payload["tensors"]
    if manifest.get("schema") != PACKET_SCHEMA:
        raise ValueError("unknown block packet schema")
    layout = manifest["layout"]
    info = engine if engine is not None else engine_info()
    if layout.get("engine", {}).get("revision") != info["revision"]:
        raise ValueError("block packet engine revision mismatch")
    names = set(manifest["packet_sha256"])
    if set(tensors) != names:
        raise ValueError("block packet tensor set mismatch")
    for name in names:
        if digest(tensors[name]) != manifest["packet_sha256"][name] or list(tensors[name].stride()) != manifest["strides"][name]:
            raise ValueError("block packet tensor checksum or layout mismatch: " + name)
    dev = model.device
    packet = {name: tensors[f"packet.{name}"].to(dev) for name in PACKET_TENSORS}
    packet["rotary"] = tuple(tensors[f"packet.rotary.{i}"].to(dev) for i in range(layout["rotary"]))
    packet["shape"] = tuple(tuple(s) for s in layout["shape"])
    packet.update(layout["xdit"])
    if "text_lens" in layout:
        packet["text_lens"] = list(layout["text_lens"])
    return model.resolve_packet(packet)
