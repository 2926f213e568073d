"""The attention call surfaces (backend plugin and SD3.5 varlen slot) on the GPU
against the oracle.  Shapes follow the reference's own dispatch test
(tests/python/test_domain_block_executor.py:861-919): joint cu [0, 7, 19] and
image-only cu [0, 4, 13] with 2 heads."""
import math

import pytest
import torch

from oracle import common as oc
from tests.helpers import assert_close, bf, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _api():
    from ditserve_amd import attention
    return attention


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("sq,sk", [(77, 77), (300, 512), (1, 65)])
def test_backend_dense_bhsd_out_and_lse(d, sq, sk):
    api = _api()
    b, h = 2, 3
    q, k, v = bf(randn((b, h, sq, d), 1)), bf(randn((b, h, sk, d), 2)), bf(randn((b, h, sk, d), 3))
    out, lse = api.ditk_attention(q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16), v.to(DEV, torch.bfloat16),
                                  api.AttnCall())
    assert out.shape == (b, h, sq, d) and lse.shape == (b, h, sq)
    for i in range(b):
        ref, ref_lse = oc.sdpa_lse(q[i], k[i], v[i])
        assert_close(out[i].float().cpu(), ref, 0.9999, 1e-2, "plugin out")
        assert torch.allclose(lse[i].cpu(), ref_lse, atol=2e-3, rtol=1e-4)


def test_backend_key_side_varlen_packing():
    """VarlenPacking selects surviving keys per batch (trailing pad keys dropped)."""
    api = _api()
    b, h, s, d = 2, 2, 96, 128
    valid = [70, 96]
    q, k, v = bf(randn((b, h, s, d), 4)), bf(randn((b, h, s, d), 5)), bf(randn((b, h, s, d), 6))
    idx = torch.cat([torch.arange(valid[0]), s + torch.arange(valid[1])]).to(DEV)
    cu_k = torch.tensor([0, valid[0], valid[0] + valid[1]], dtype=torch.int32, device=DEV)
    call = api.AttnCall(varlen=api.VarlenPacking(idx, cu_k, max(valid)))
    out, _ = api.ditk_attention(q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16), v.to(DEV, torch.bfloat16), call)
    for i in range(b):
        ref = oc.sdpa(q[i], k[i, :, :valid[i]], v[i, :, :valid[i]])
        assert_close(out[i].float().cpu(), ref, 0.9999, 1e-2, f"varlen batch {i}")


def test_backend_rejects_unsupported_calls():
    api = _api()
    x = torch.zeros((1, 2, 8, 128), dtype=torch.bfloat16, device=DEV)
    assert "causal" in api.unmet(x, x, x, api.AttnCall(is_causal=True))
    assert "dropout" in api.unmet(x, x, x, api.AttnCall(dropout_p=0.1))
    assert "bfloat16" in api.unmet(x.half(), x.half(), x.half(), api.AttnCall())
    y = torch.zeros((1, 2, 8, 96), dtype=torch.bfloat16, device=DEV)
    assert "head dimension" in api.unmet(y, y, y, api.AttnCall())
    with pytest.raises(NotImplementedError):
        api.ditk_attention(x, x, x, api.AttnCall(is_causal=True))


@pytest.mark.parametrize("cu,d", [([0, 7, 19], 64), ([0, 4, 13], 64), ([0, 4429, 8858, 10215], 64),
                                  ([0, 1, 300, 301], 128)])
def test_sd35_varlen_slot(cu, d):
    """flash_attn_varlen_func(q, k, v, cu_q, cu_k, max_q, max_k) == per-segment SDPA
    (the reference's fake slot, test_domain_block_executor.py:869-883)."""
    api = _api()
    h, t = 2, cu[-1]
    q, k, v = bf(randn((t, h, d), 7)), bf(randn((t, h, d), 8)), bf(randn((t, h, d), 9))
    cu_t = torch.tensor(cu, dtype=torch.int32, device=DEV)
    mx = max(b - a for a, b in zip(cu, cu[1:]))
    out = api.flash_attn_varlen_func(q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16), v.to(DEV, torch.bfloat16),
                                     cu_t, cu_t, mx, mx, dropout_p=0.0, causal=False)
    assert out.shape == (t, h, d) and out.dtype == torch.bfloat16
    ref = oc.varlen_attention(q, k, v, cu, cu)
    assert_close(out.float().cpu(), ref, 0.9999, 1e-2, f"slot {cu}")
    with pytest.raises(NotImplementedError):
        api.flash_attn_varlen_func(q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16), v.to(DEV, torch.bfloat16),
                                   cu_t, cu_t, mx, mx, causal=True)
    _ = math


@pytest.mark.parametrize("bad,clamped", [([0, 200, 400], [0, 200, 300]),      # past the token count
                                         ([0, 250, 100, 300], [0, 250, 250, 300]),  # decreasing
                                         ([5, 100, 300], [0, 100, 300]),       # not starting at 0
                                         ([0, 100, 299], [0, 100, 299])])      # short of the token count
def test_sd35_varlen_slot_invalid_tables_are_clamped_and_reported(bad, clamped):
    """A caller's device cu table that is not valid is copied, clamped into [0, T]
    and made nondecreasing, on the GPU before any kernel reads it, so no kernel
    leaves the tensors; the sticky status reports it: check_tables() after a sync,
    and the next call once the check has finished.  Valid calls then run as before."""
    api = _api()
    from ditserve_amd import ops
    from ditserve_amd._lib import DitkError
    h, d, t = 2, 64, 300
    q, k, v = bf(randn((t, h, d), 10)), bf(randn((t, h, d), 11)), bf(randn((t, h, d), 12))
    qd, kd, vd = (x.to(DEV, torch.bfloat16) for x in (q, k, v))
    good = torch.tensor([0, 120, 300], dtype=torch.int32, device=DEV)
    badt = torch.tensor(bad, dtype=torch.int32, device=DEV)
    api.flash_attn_varlen_func(qd, kd, vd, good, good, 180, 180)
    api.check_tables()                                   # nothing to report
    seg = ops.Segments.from_device(badt, t)
    assert seg.dev.tolist() == clamped and badt.tolist() == bad
    with pytest.raises(DitkError):
        api.check_tables()
    api.check_tables()                                   # reported once
    with pytest.raises(DitkError):
        # reported by the first table check that starts after the bad table's
        # check has finished: the bad call's key table, or the next call
        api.flash_attn_varlen_func(qd, kd, vd, badt, badt, 300, 300)
        torch.cuda.synchronize()
        api.flash_attn_varlen_func(qd, kd, vd, good, good, 180, 180)
    out = api.flash_attn_varlen_func(qd, kd, vd, good, good, 180, 180)
    api.check_tables()
    assert_close(out.float().cpu(), oc.varlen_attention(q, k, v, [0, 120, 300], [0, 120, 300]), 0.9999, 1e-2,
                 "after report")


def test_cu_table_check_across_chunks():
    """Tables longer than the check kernel's 256-entry chunk: a valid 600-segment
    table is copied unchanged and not reported; a dip at entry 300 is clamped with
    the running max carried over from the earlier chunks."""
    from ditserve_amd import ops
    from ditserve_amd._lib import DitkError
    cu = [3 * i for i in range(601)]
    seg = ops.Segments.from_device(torch.tensor(cu, dtype=torch.int32, device=DEV), cu[-1])
    assert seg.dev.tolist() == cu
    ops.check_tables()
    dip = list(cu)
    dip[300] = 5
    seg = ops.Segments.from_device(torch.tensor(dip, dtype=torch.int32, device=DEV), cu[-1])
    assert seg.dev.tolist() == cu[:300] + [cu[299]] + cu[301:]
    with pytest.raises(DitkError):
        ops.check_tables()


def test_backend_uniform_tables_are_cached():
    """ditk_attention without key packing reuses one device table per shape."""
    api = _api()
    from ditserve_amd import ops
    x = torch.zeros((2, 2, 77, 64), dtype=torch.bfloat16, device=DEV)
    api.ditk_attention(x, x, x)
    a = ops.Segments.uniform(2, 77, DEV)
    api.ditk_attention(x, x, x)
    assert ops.Segments.uniform(2, 77, DEV) is a and a.dev.tolist() == [0, 77, 154]
