"""Attention entry points with the reference's call contracts, on the ditk
varlen flash kernel (bf16, head_dim 64/128, non-causal, no dropout).

1. Attention-backend plugin (workers/xfuser/core/attention/spec.py:88-106,283-304):
   ``ditk_attention(query, key, value, call) -> (out, lse)`` over BHSD tensors,
   ``call`` an ``AttnCall``-shaped object (dropout_p, is_causal, varlen).  Key-side
   varlen packing (``VarlenPacking``: indices_k / cu_seqlens_k / max_seqlen_k,
   spec.py:63-85) is honoured by gathering the surviving keys.
   ``unmet(query, key, value, call)`` returns the reason a call is refused, or
   None — the backend's ``accepts`` facts (spec.py:244-246).
2. SD3.5 varlen slot (workers/ditserve/models/sd35_batch.py:19-119, called at
   :448-486): ``flash_attn_varlen_func(q, k, v, cu_q, cu_k, max_q, max_k,
   dropout_p=0.0, causal=False) -> out`` on packed [T, H, D] tensors with int32
   device cu_seqlens.  No host synchronisation: cu tables stay on the device.

Device cu_seqlens tables from callers are checked on the GPU before any kernel
reads them (ops.Segments.from_device): an invalid table is clamped into bounds
and reported by the next call after the check has finished, or by
``check_tables()``.  BHSD calls without key packing reuse cached per-shape
segment tables, so a steady call uploads nothing.
"""
import dataclasses
from typing import Optional

import torch

from . import ops

HEAD_DIMS = (64, 128)
REQUIRES_ARCH = "gfx950"


@dataclasses.dataclass(frozen=True)
class VarlenPacking:
    """Key-side packing: rows ``indices_k`` of the flattened B*S keys survive;
    ``cu_seqlens_k`` / ``max_seqlen_k`` describe the packed result."""

    indices_k: torch.Tensor
    cu_seqlens_k: torch.Tensor
    max_seqlen_k: int

    @classmethod
    def from_kwargs(cls, attention_kwargs):
        """The packing a model put in its attention kwargs (keys ``indices_k``,
        ``cu_seqlens_k``, ``max_seqlen_k``; spec.py:74-85), or None without
        ``indices_k``."""
        kw = attention_kwargs or {}
        if kw.get("indices_k") is None:
            return None
        return cls(kw["indices_k"], kw["cu_seqlens_k"], kw["max_seqlen_k"])


@dataclasses.dataclass
class AttnCall:
    """What a backend needs about one call besides q/k/v."""

    dropout_p: float = 0.0
    is_causal: bool = False
    varlen: Optional[VarlenPacking] = None
    # sequence-parallel degrees (spec.py:99-100): a dense backend computes the
    # attention of the heads and keys it is handed whatever they are
    ulysses_world_size: int = 1
    ring_world_size: int = 1
    attention_kwargs: dict = dataclasses.field(default_factory=dict)


def unmet(query, key, value, call) -> Optional[str]:
    """Reason this backend cannot serve the call, or None."""
    if getattr(call, "is_causal", False):
        return "does not support causal masking"
    if getattr(call, "dropout_p", 0.0) not in (None, 0.0):
        return "does not support attention dropout"
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.dtype != torch.bfloat16:
            return f"supports bfloat16 only, got {name} dtype {t.dtype}"
        if t.device.type != "cuda":
            return f"needs device tensors, got {name} on {t.device}"
    if query.shape[-1] not in HEAD_DIMS or key.shape[-1] != query.shape[-1] or value.shape[-1] != query.shape[-1]:
        return f"supports head dimension 64, 128 only, got {query.shape[-1]}"
    if query.shape[1] != key.shape[1] or key.shape[1] != value.shape[1]:
        return "supports MHA only (equal query and key/value head counts)"
    if call is not None and (getattr(call, "attention_kwargs", None) or {}).get("attn_mask") is not None:
        return "does not support attn_mask"
    return None


def _rows(x):
    """[B, H, S, D] -> contiguous [B*S, H*D]."""
    b, h, s, d = x.shape
    return x.transpose(1, 2).reshape(b * s, h * d).contiguous()


def ditk_attention(query, key, value, call=None):
    """BHSD attention: returns (out [B, H, Sq, D] bf16, lse [B, H, Sq] fp32, natural log)."""
    call = call if call is not None else AttnCall()
    reason = unmet(query, key, value, call)
    if reason is not None:
        raise NotImplementedError(f"DITK {reason}")
    b, h, sq, d = query.shape
    sk = key.shape[2]
    q = _rows(query)
    if call.varlen is not None:
        kv_k, kv_v = _rows(key), _rows(value)
        idx = call.varlen.indices_k
        k, v = kv_k.index_select(0, idx), kv_v.index_select(0, idx)
        seg_k = ops.Segments.from_device(call.varlen.cu_seqlens_k.to(torch.int32), k.shape[0])
        if seg_k.nseg != b:
            raise ValueError(f"varlen packing describes {seg_k.nseg} batches, query has {b}")
    else:
        k, v = _rows(key), _rows(value)
        seg_k = ops.Segments.uniform(b, sk, query.device)
    seg_q = ops.Segments.uniform(b, sq, query.device)
    out, lse = ops.flash_attn_varlen(q, k, v, seg_q, seg_k, h, d, return_lse=True)
    out = out.view(b, sq, h, d).transpose(1, 2)
    lse = lse.view(h, b, sq).permute(1, 0, 2)
    return out, lse


def flash_attn_varlen_func(q, k, v, cu_q, cu_k, max_q, max_k, dropout_p=0.0, causal=False):
    """Packed varlen attention: q [Tq, H, D], k/v [Tk, H, D] bf16, cu_q/cu_k int32
    [nseg+1] on the device; segment m's queries attend to its keys only."""
    if causal:
        raise NotImplementedError("DITK does not support causal masking")
    if dropout_p not in (None, 0.0):
        raise NotImplementedError("DITK does not support attention dropout")
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k, v must be [T, H, D]")
    tq, h, d = q.shape
    if cu_q.numel() != cu_k.numel():
        raise ValueError("cu_seqlens_q and cu_seqlens_k must have the same length")
    seg_q = ops.Segments.from_device(cu_q.to(torch.int32), tq)
    seg_k = ops.Segments.from_device(cu_k.to(torch.int32), k.shape[0])
    out = ops.flash_attn_varlen(q.reshape(tq, h * d), k.reshape(k.shape[0], h * d),
                                v.reshape(v.shape[0], h * d).contiguous(), seg_q, seg_k, h, d)
    return out.view(tq, h, d)


def check_tables(device=None):
    """Wait for the device and raise if a cu_seqlens table passed to these entry
    points since the last report was invalid (see ops.Segments.from_device)."""
    ops.check_tables(device)
