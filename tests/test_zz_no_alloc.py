"""The allocation-free attention entry point (ditk_flash_attn_varlen_noalloc),
called through the C ABI, against the existing entry points it replaces for
callers that cannot allocate (ditk_transpose_v into a caller buffer +
ditk_flash_attn_varlen): bitwise equal outputs and LSE on two calls in a row,
the second smaller, and a clear rejection above the scratch limit."""
import ctypes
import math

import pytest
import torch

from tests.helpers import randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCRATCH_BYTES = 64 << 20  # DITK_NOALLOC_SCRATCH_BYTES


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _case(counts_q, counts_k, heads, hd, seed):
    width = heads * hd
    cu_q = [0]
    for n in counts_q:
        cu_q.append(cu_q[-1] + n)
    cu_k = [0]
    for n in counts_k:
        cu_k.append(cu_k[-1] + n)
    q = randn((cu_q[-1], width), seed).to(DEV, torch.bfloat16)
    kv = randn((cu_k[-1], 2 * width), seed + 1).to(DEV, torch.bfloat16)
    return q, kv[:, :width], kv[:, width:], torch.tensor(cu_q, dtype=torch.int32, device=DEV), \
        torch.tensor(cu_k, dtype=torch.int32, device=DEV)


def _existing(lib, q, k, v, cu_q, cu_k, heads, hd, scale):
    Tq, Tk, nseg = q.shape[0], k.shape[0], cu_q.numel() - 1
    cols = lib.ditk_vt_columns(Tk, nseg)
    vt = torch.empty((heads, hd, cols), dtype=torch.bfloat16, device=DEV)
    o = torch.empty((Tq, heads * hd), dtype=torch.bfloat16, device=DEV)
    lse = torch.empty((heads, Tq), dtype=torch.float32, device=DEV)
    assert lib.ditk_transpose_v(_p(v), v.stride(0), _p(vt), cols, Tk, heads, hd, _p(cu_k), nseg, _stream()) == 0
    assert lib.ditk_flash_attn_varlen(_p(q), q.stride(0), _p(k), k.stride(0), _p(vt), cols, _p(o), o.stride(0),
                                      _p(lse), Tq, _p(cu_q), _p(cu_k), nseg, Tq, heads, hd, ctypes.c_float(scale),
                                      _stream()) == 0
    return o, lse


def _noalloc(lib, q, k, v, cu_q, cu_k, heads, hd, scale):
    Tq, Tk, nseg = q.shape[0], k.shape[0], cu_q.numel() - 1
    o = torch.empty((Tq, heads * hd), dtype=torch.bfloat16, device=DEV)
    lse = torch.empty((heads, Tq), dtype=torch.float32, device=DEV)
    rc = lib.ditk_flash_attn_varlen_noalloc(_p(q), q.stride(0), _p(k), k.stride(0), _p(v), v.stride(0), _p(o),
                                            o.stride(0), _p(lse), Tq, _p(cu_q), _p(cu_k), nseg, Tq, Tk, heads, hd,
                                            ctypes.c_float(scale), _stream())
    assert rc == 0, lib.ditk_last_error().decode()
    return o, lse


def test_noalloc_matches_existing_entry_point_twice():
    from ditserve_amd import _lib
    lib = _lib.load()
    cases = [([700, 1300, 33], [700, 1300, 33], 12, 128, 1),   # self-attention, 3 ragged segments
             ([300, 77], [512, 512], 4, 64, 2)]                # cross-attention shape, smaller, head_dim 64
    for counts_q, counts_k, heads, hd, seed in cases:
        q, k, v, cu_q, cu_k = _case(counts_q, counts_k, heads, hd, seed)
        scale = 1.0 / math.sqrt(hd)
        ref_o, ref_lse = _existing(lib, q, k, v, cu_q, cu_k, heads, hd, scale)
        got_o, got_lse = _noalloc(lib, q, k, v, cu_q, cu_k, heads, hd, scale)
        torch.cuda.synchronize()
        assert torch.isfinite(got_o.float()).all()
        assert torch.equal(got_o, ref_o) and torch.equal(got_lse, ref_lse)


def test_noalloc_rejects_inputs_above_the_scratch_limit():
    from ditserve_amd import _lib
    lib = _lib.load()
    heads, hd = 12, 128
    tk = SCRATCH_BYTES // (heads * hd * 2) + 64  # one tile more than the scratch holds
    q = torch.zeros((64, heads * hd), dtype=torch.bfloat16, device=DEV)
    kv = torch.zeros((tk, heads * hd), dtype=torch.bfloat16, device=DEV)
    o = torch.empty_like(q)
    cu_q = torch.tensor([0, 64], dtype=torch.int32, device=DEV)
    cu_k = torch.tensor([0, tk], dtype=torch.int32, device=DEV)
    rc = lib.ditk_flash_attn_varlen_noalloc(_p(q), q.stride(0), _p(kv), kv.stride(0), _p(kv), kv.stride(0), _p(o),
                                            o.stride(0), None, 0, _p(cu_q), _p(cu_k), 1, 64, tk, heads, hd,
                                            ctypes.c_float(0.1), _stream())
    assert rc != 0 and b"scratch" in lib.ditk_last_error()
