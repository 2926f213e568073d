"""GPU parity of each ditk kernel against the CPU oracle (fp32 on the same
bf16-rounded inputs).  Tolerances are stated per test; integer/index work is
checked bit-exactly, packed-vs-solo runs bitwise."""
import math

import pytest
import torch

from oracle import common as oc
from oracle import wan as ow
from tests.helpers import assert_close, bf, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ops():
    from ditserve_amd import ops
    return ops


def _seg(cu):
    return _ops().Segments(cu, DEV)


# --------------------------------------------------------------------------- GEMM
GEMM_CASES = [(1000, 1536, 1536), (256, 4608, 1536), (77, 64, 1536), (513, 384, 8960), (33, 1536, 64),
              (300, 512, 96),  # K % 64 == 32: the 32-k stage path
              (4000, 4104, 1536),  # 16 x 22 256x192 tiles (two rounds, fewer than 16 x 17 256x256), ragged M and N
              (4000, 4096, 1536)]  # 16 x 16 256x256 tiles (one round; 256x192 would take two), ragged M


@pytest.mark.parametrize("M,N,K", GEMM_CASES)
@pytest.mark.parametrize("epi", ["bias", "gelu", "f32", "silu"])
def test_gemm_epilogues(M, N, K, epi):
    ops = _ops()
    a, w, b = bf(randn((M, K), 1)), bf(randn((N, K), 2, 0.02)), bf(randn((N,), 3, 0.1))
    out = ops.linear(a.to(DEV, torch.bfloat16), w.to(DEV, torch.bfloat16), b.to(DEV), epi).float().cpu()
    ref = oc.linear(a, w, b)
    if epi == "gelu":
        ref = oc.gelu_tanh(ref)
    elif epi == "silu":
        ref = oc.silu(ref)
    # bf16 output rounding bounds the error (2^-9 relative per element)
    assert_close(out, ref, cos_min=0.99999, rel_max=5e-3, label=f"gemm {epi} {M}x{N}x{K}")


@pytest.mark.parametrize("epi", ["gate_res", "res"])
def test_gemm_residual_epilogues(epi):
    ops = _ops()
    M, N, K = 700, 1536, 1536
    cu = [0, 300, 650, 700]
    a, w, b = bf(randn((M, K), 4)), bf(randn((N, K), 5, 0.02)), bf(randn((N,), 6, 0.1))
    r = bf(randn((M, N), 7))
    gate = randn((3, N), 8)
    seg = _seg(cu)
    out = ops.linear(a.to(DEV, torch.bfloat16), w.to(DEV, torch.bfloat16), b.to(DEV), epi,
                     residual=r.to(DEV, torch.bfloat16), gate=gate.to(DEV), segments=seg).float().cpu()
    y = oc.linear(a, w, b)
    if epi == "gate_res":
        g = torch.cat([gate[i].expand(cu[i + 1] - cu[i], N) for i in range(3)])
        ref = r + y * g
    else:
        ref = r + y
    assert_close(out, ref, cos_min=0.99999, rel_max=5e-3, label=epi)


def test_gemm_rows_independent_of_packing():
    """A row's result does not depend on M or on where the row sits (bitwise)."""
    ops = _ops()
    K, N = 1536, 1536
    a = randn((900, K), 9).to(DEV, torch.bfloat16)
    w = randn((N, K), 10, 0.02).to(DEV, torch.bfloat16)
    b = randn((N,), 11).to(DEV)
    full = ops.linear(a, w, b)
    part = ops.linear(a[313:777].contiguous(), w, b)
    assert torch.equal(full[313:777], part)


@pytest.mark.parametrize("epi", ["bias", "gelu", "f32", "gate_res", "res", "silu"])
@pytest.mark.parametrize("K,N", [(1536, 4096), (1536, 1536), (96, 2048), (4160, 2048), (4160, 1024)])
def test_gemm_tile_configs_agree(epi, K, N):
    """Large M runs large workgroup tiles, a few hundred rows the 64x128 ones; all
    use the same MFMA, k order and epilogue arithmetic, so rows computed in either
    are bitwise equal.  At M = 8192 on 256 CUs: N = 4096 and (K = 4160, N = 2048)
    take the one-wave-per-SIMD 256x256 kernel, N = 1536 and (4160, 1024) its
    256x192 form (fewer tile rounds), K = 96 (an odd number of 32-k stages) and
    the fp32 epilogue the 8-wave kernel."""
    ops = _ops()
    M = 8192
    a = randn((M, K), 40).to(DEV, torch.bfloat16)
    w = randn((N, K), 41, 0.02).to(DEV, torch.bfloat16)
    b = randn((N,), 42).to(DEV)
    kw = {}
    if epi == "gate_res":
        kw = dict(residual=randn((M, N), 43).to(DEV, torch.bfloat16), gate=randn((2, N), 44).to(DEV),
                  segments=_seg([0, 5000, M]))
    elif epi == "res":
        kw = dict(residual=randn((M, N), 43).to(DEV, torch.bfloat16))
    full = ops.linear(a, w, b, epi, **kw)
    lo, hi = 4700, 5333  # 633 rows across the segment boundary: at most 3 x 16 large tiles, so small ones run
    if epi == "gate_res":
        kw = dict(residual=kw["residual"][lo:hi].contiguous(), gate=kw["gate"], segments=_seg([0, 5000 - lo, hi - lo]))
    elif epi == "res":
        kw = dict(residual=kw["residual"][lo:hi].contiguous())
    part = ops.linear(a[lo:hi].contiguous(), w, b, epi, **kw)
    assert torch.equal(full[lo:hi], part)


@pytest.mark.parametrize("epi", ["bias", "res", "gate_res", "gelu"])
def test_gemm_persistent_tiles_agree(epi):
    """M = 20000, N = K = 1536: 474 large tiles on at most 256 persistent
    workgroups (some take two), the last tile row ragged (20000 = 78 x 256 + 32).
    Rows computed there equal, bitwise, the same rows computed alone by the
    small-tile kernel: a slice ending at the last row and one across tile rows."""
    ops = _ops()
    M, N, K = 20000, 1536, 1536
    a = randn((M, K), 50).to(DEV, torch.bfloat16)
    w = randn((N, K), 51, 0.02).to(DEV, torch.bfloat16)
    b = randn((N,), 52).to(DEV)
    r = randn((M, N), 53).to(DEV, torch.bfloat16)
    gate = randn((2, N), 54).to(DEV)
    cut = 12345

    def run(lo, hi):
        kw = {}
        if epi == "gate_res":
            kw = dict(residual=r[lo:hi].contiguous(), gate=gate,
                      segments=_seg([0, min(max(cut - lo, 0), hi - lo), hi - lo]))
        elif epi == "res":
            kw = dict(residual=r[lo:hi].contiguous())
        return ops.linear(a[lo:hi].contiguous(), w, b, epi, **kw)

    full = run(0, M)
    for lo, hi in ((M - 633, M), (cut - 300, cut + 333)):
        assert torch.equal(full[lo:hi], run(lo, hi)), (epi, lo, hi)


@pytest.mark.parametrize("epi", ["bias", "res", "gate_res", "gelu"])
def test_gemm_short_tile_row_split_agrees(epi):
    """M = 10792 = 42 x 256 + 40, N = 4608, K = 1536: 43 x 18 = 774 large tiles
    are 4 rounds of 256 CUs but 42 x 18 = 756 are 3, so the 40 rows of the last
    tile row go to the small-tile kernel in a second launch (rows offset into the
    gated residual's segments: a segment ends 22 rows into them).  The same rows
    inside an 11008-row product (43 whole tile rows, one launch) are equal
    bitwise, and the product is close to an fp32 reference."""
    ops = _ops()
    M, N, K, M2 = 10792, 4608, 1536, 11008
    a = randn((M2, K), 60).to(DEV, torch.bfloat16)
    w = randn((N, K), 61, 0.02).to(DEV, torch.bfloat16)
    b = randn((N,), 62).to(DEV)
    r = randn((M2, N), 63).to(DEV, torch.bfloat16)
    gate = randn((4, N), 64).to(DEV)
    cut = [0, 5000, 10774, M, M2]

    def run(m):
        kw = {}
        if epi == "gate_res":
            nseg = 3 if m == M else 4
            kw = dict(residual=r[:m].contiguous(), gate=gate[:nseg], segments=_seg(cut[:nseg + 1]))
        elif epi == "res":
            kw = dict(residual=r[:m].contiguous())
        return ops.linear(a[:m].contiguous(), w, b, epi, **kw)

    y = run(M)
    assert torch.equal(y, run(M2)[:M]), epi
    rows = torch.arange(M - 300, M, device=DEV)
    ref = a[rows].float() @ w.float().t() + b
    if epi == "gelu":
        ref = torch.nn.functional.gelu(ref, approximate="tanh")
    elif epi == "res":
        ref = r[rows].float() + ref.bfloat16().float()
    elif epi == "gate_res":
        seg = torch.bucketize(rows, torch.tensor(cut[1:4], device=DEV), right=True)
        ref = r[rows].float() + ref.bfloat16().float() * gate[seg]
    assert_close(y[rows].float(), ref, 0.999, 1e-2, f"split {epi}")


@pytest.mark.parametrize("epi", ["gate_res", "bias", "gelu", "res", "silu"])
@pytest.mark.parametrize("M0,M1,N,K", [(8192, 666, 1536, 1536),   # one launch: 192 + 18 tiles = one round
                                       (666, 8192, 1536, 6144),   # the same, text first, long K
                                       (8192, 666, 4608, 1536)])  # two launches: the text tiles add a round
def test_gemm_pair_matches_separate(epi, M0, M1, N, K):
    """ditk_gemm_pair (SD3.5's image and text projections of one block) returns,
    bitwise, what two ditk_gemm calls return, in one launch or two; each product
    keeps its own gate rows and segments (2 image, 2 text)."""
    ops = _ops()

    def prob(M, seed):
        p = dict(x=randn((M, K), seed).to(DEV, torch.bfloat16), w=randn((N, K), seed + 1, 0.02).to(DEV, torch.bfloat16),
                 b=randn((N,), seed + 2).to(DEV))
        if epi in ("gate_res", "res"):
            p["residual"] = randn((M, N), seed + 3).to(DEV, torch.bfloat16)
        if epi == "gate_res":
            p["gate"] = randn((2, N), seed + 4).to(DEV)
            p["segments"] = _seg([0, M // 2 + 7, M])
        return p

    p0, p1 = prob(M0, 70), prob(M1, 80)
    y0, y1 = ops.linear_pair(p0, p1, epi)
    assert torch.equal(y0, ops.linear(epilogue=epi, **p0)), "first product"
    assert torch.equal(y1, ops.linear(epilogue=epi, **p1)), "second product"
    with pytest.raises(ValueError):
        ops.linear_pair(p0, dict(x=p1["x"][:, :K - 32].contiguous(), w=p1["w"][:, :K - 32].contiguous()), epi)


@pytest.mark.parametrize("epi", ["gate_res", "res"])
def test_gemm_pair_in_place_matches_separate(epi):
    """SD3.5's block calls the pair in place (out = residual = h for the image rows,
    out = residual = c for the text rows).  At (8192, 666, 1536, 1536) the pair runs
    in one launch; each product's in-place result equals, bitwise, an in-place
    ditk_gemm on a copy.  Overlap between the products is refused on the host."""
    ops = _ops()
    N = K = 1536

    def prob(M, seed):
        p = dict(x=randn((M, K), seed).to(DEV, torch.bfloat16), w=randn((N, K), seed + 1, 0.02).to(DEV, torch.bfloat16),
                 b=randn((N,), seed + 2).to(DEV), residual=randn((M, N), seed + 3).to(DEV, torch.bfloat16))
        if epi == "gate_res":
            p["gate"] = randn((2, N), seed + 4).to(DEV)
            p["segments"] = _seg([0, M // 2 + 7, M])
        return p

    p0, p1 = prob(8192, 90), prob(666, 95)
    ref0 = p0["residual"].clone()
    ref1 = p1["residual"].clone()
    ops.linear(epilogue=epi, **dict(p0, residual=ref0, out=ref0))
    ops.linear(epilogue=epi, **dict(p1, residual=ref1, out=ref1))
    p0["out"], p1["out"] = p0["residual"], p1["residual"]
    y0, y1 = ops.linear_pair(p0, p1, epi)
    assert y0.data_ptr() == p0["residual"].data_ptr() and y1.data_ptr() == p1["residual"].data_ptr()
    assert torch.equal(y0, ref0), "image rows in place"
    assert torch.equal(y1, ref1), "text rows in place"
    with pytest.raises(ValueError):   # product 1 reads rows product 0 writes
        ops.linear_pair(p0, dict(p1, x=p0["residual"][:666]), epi)


def test_gemm_stage_depths_agree():
    """K % 64 == 0 runs 64-k LDS stages, otherwise 32-k stages; the MFMA k order is
    the same, so zero-padding K by 32 (forcing the 32-k path) changes no bit."""
    ops = _ops()
    M, N, K = 600, 768, 1536
    a = randn((M, K), 30).to(DEV, torch.bfloat16)
    w = randn((N, K), 31, 0.02).to(DEV, torch.bfloat16)
    b = randn((N,), 32).to(DEV)
    a_pad = torch.cat([a, torch.zeros((M, 32), dtype=a.dtype, device=DEV)], 1).contiguous()
    w_pad = torch.cat([w, randn((N, 32), 33).to(DEV, torch.bfloat16)], 1).contiguous()
    assert torch.equal(ops.linear(a, w, b), ops.linear(a_pad, w_pad, b))
    assert torch.equal(ops.linear(a, w, b, "f32"), ops.linear(a_pad, w_pad, b, "f32"))


# --------------------------------------------------------------------------- AdaLN
@pytest.mark.parametrize("D", [1536, 3072, 64, 5120, 6144])  # 5120: Wan2.1-14B; 6144: the widest row
def test_adaln_modulated_layernorm(D):
    ops = _ops()
    cu = [0, 37, 300, 301, 512]
    T = cu[-1]
    x = bf(randn((T, D), 12, 3.0) + 0.5)
    shift, scale = randn((4, D), 13), randn((4, D), 14)
    out = ops.adaln(x.to(DEV, torch.bfloat16), shift.to(DEV), scale.to(DEV), _seg(cu)).float().cpu()
    ref = torch.empty(T, D)
    for m in range(4):
        s0, s1 = cu[m], cu[m + 1]
        ref[s0:s1] = oc.layer_norm(x[s0:s1]) * (1 + scale[m]) + shift[m]
    assert_close(out, ref, cos_min=0.99999, rel_max=5e-3, label=f"adaln D={D}")


def test_adaln_affine_and_rms():
    ops = _ops()
    T, D = 333, 1536
    x = bf(randn((T, D), 15, 2.0))
    w, b = randn((D,), 16, 0.1) + 1, randn((D,), 17, 0.1)
    out = ops.adaln(x.to(DEV, torch.bfloat16), weight=w.to(DEV), bias=b.to(DEV)).float().cpu()
    assert_close(out, oc.layer_norm(x, 1e-6, w, b), cos_min=0.99999, rel_max=5e-3, label="ln affine")
    xd = x.to(DEV, torch.bfloat16)
    ops.adaln(xd, weight=w.to(DEV), kind="rms", out=xd)  # in place
    assert_close(xd.float().cpu(), oc.rms_norm(x, w), cos_min=0.99999, rel_max=5e-3, label="rms")


# --------------------------------------------------------------------------- QK norm + RoPE
@pytest.mark.parametrize("D", [1536, 5120])  # Wan2.1-1.3B and -14B (40 heads)
def test_qk_norm_rope_matches_oracle(D):
    ops = _ops()
    from ditserve_amd.wan import rope_axis_pairs, rope_tables
    Dh = 128
    H = D // Dh
    grids = [(3, 5, 7), (2, 4, 6), (1, 1, 1)]
    counts = [f * h * w for f, h, w in grids]
    cu = [0, counts[0], counts[0] + counts[1], sum(counts)]
    T = cu[-1]
    q, k = bf(randn((T, D), 18, 2.0)), bf(randn((T, D), 19, 2.0))
    wq, wk = bf(randn((D,), 20, 0.1) + 1), bf(randn((D,), 21, 0.1) + 1)
    seg = _seg(cu)
    cos_t, sin_t = rope_tables(Dh, 1024, 10000.0, DEV)
    tp, hp, _ = rope_axis_pairs(Dh)
    rope = ops.Rope(cos_t, sin_t, grids, seg, tp, hp)
    qd, kd = q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16)
    ops.qk_norm_rope_(qd, kd, wq.to(DEV), wk.to(DEV), Dh, rope=rope)
    for m, g in enumerate(grids):
        s0, s1 = cu[m], cu[m + 1]
        cos, sin = ow.rope_freqs(g, Dh)
        rq, rk = ow.qk_norm_rope(q[s0:s1], k[s0:s1], wq, wk, cos, sin, H)
        assert_close(qd[s0:s1].float().cpu(), rq.flatten(1), cos_min=0.99999, rel_max=5e-3, label="q")
        assert_close(kd[s0:s1].float().cpu(), rk.flatten(1), cos_min=0.99999, rel_max=5e-3, label="k")


def test_qk_norm_rope_out_of_place_bitwise():
    """The out-of-place entry writes exactly what the in-place one leaves, into
    strided column slices of another buffer, and leaves its inputs untouched;
    rope and per-head forms."""
    ops = _ops()
    from ditserve_amd.wan import rope_axis_pairs, rope_tables
    D, Dh = 1536, 128
    grids = [(2, 3, 5), (1, 4, 4)]
    cu = [0, 30, 46]
    T = cu[-1]
    q = randn((T, D), 60, 2.0).to(DEV, torch.bfloat16)
    k = randn((T, D), 61, 2.0).to(DEV, torch.bfloat16)
    wq, wk = (randn((D,), 62, 0.1) + 1).to(DEV), (randn((D,), 63, 0.1) + 1).to(DEV)
    cos_t, sin_t = rope_tables(Dh, 1024, 10000.0, DEV)
    tp, hp, _ = rope_axis_pairs(Dh)
    rope = ops.Rope(cos_t, sin_t, grids, _seg(cu), tp, hp)
    for per_head, rp in ((False, rope), (True, None)):
        qi, ki = q.clone(), k.clone()
        ops.qk_norm_rope_(qi, ki, wq, wk, Dh, per_head=per_head, rope=rp)
        buf = torch.zeros((T, 3 * D), dtype=torch.bfloat16, device=DEV)
        qo, ko = ops.qk_norm_rope_(q, k, wq, wk, Dh, per_head=per_head, rope=rp, out=(buf[:, :D], buf[:, 2 * D:]))
        assert torch.equal(qo, qi) and torch.equal(ko, ki)
        assert torch.equal(buf[:, D:2 * D], torch.zeros_like(buf[:, D:2 * D]))
    assert torch.equal(q, randn((T, D), 60, 2.0).to(DEV, torch.bfloat16))
    assert torch.equal(k, randn((T, D), 61, 2.0).to(DEV, torch.bfloat16))


@pytest.mark.parametrize("D", [1536, 2432])  # SD3.5-Medium and -Large (38 heads of 64)
def test_qk_norm_per_head_no_rope(D):
    ops = _ops()
    T, Dh = 100, 64
    q, k = bf(randn((T, D), 22)), bf(randn((T, D), 23))
    wq, wk = bf(randn((Dh,), 24, 0.1) + 1), bf(randn((Dh,), 25, 0.1) + 1)
    qd, kd = q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16)
    ops.qk_norm_rope_(qd, kd, wq.repeat(D // Dh).to(DEV), wk.repeat(D // Dh).to(DEV), Dh, per_head=True)
    rq = oc.rms_norm(q.view(T, -1, Dh), wq).flatten(1)
    assert_close(qd.float().cpu(), rq, cos_min=0.99999, rel_max=5e-3, label="per-head q")


# --------------------------------------------------------------------------- multi-job norm launches
def test_adaln_multi_matches_single_calls():
    """One launch of several AdaLN jobs writes, per job, bitwise what a single
    adaln() call writes: modulated LayerNorms over strided [nseg, 6D] modulation
    views (image, text, the text's (scale, shift) order), a zero-row job between
    them, an in-place RMSNorm pair; mismatched kinds or widths are refused."""
    ops = _ops()
    from ditserve_amd._lib import DitkError
    D = 1536
    xi = randn((1000, D), 90, 3.0).to(DEV, torch.bfloat16)
    xt = randn((333, D), 91, 2.0).to(DEV, torch.bfloat16)
    modi, modt = randn((2, 6 * D), 92).to(DEV), randn((3, 6 * D), 93).to(DEV)
    si, st = _seg([0, 500, 1000]), _seg([0, 154, 154, 333])
    jobs = [dict(x=xi, shift=modi[:, 0:D], scale=modi[:, D:2 * D], segments=si),
            dict(x=xi[:0], weight=(randn((D,), 94, 0.1) + 1).to(DEV), out=torch.empty_like(xt)[:0]),
            dict(x=xt, shift=modt[:, D:2 * D], scale=modt[:, 0:D], segments=st, eps=1e-5),
            dict(x=xi, shift=modi[:, 3 * D:4 * D], scale=modi[:, 4 * D:5 * D], segments=si)]
    got = ops.adaln_multi(jobs)
    for j, g in zip(jobs, got):
        assert torch.equal(g, ops.adaln(**j))
    assert got[1].shape == (0, D)
    w = (randn((D,), 95, 0.1) + 1).to(DEV)
    qi, kt = xi.clone(), xt[:, :1024].clone()
    with pytest.raises(DitkError):  # ceil(D / 512) differs (3 vs 2)
        ops.adaln_multi([dict(x=qi, weight=w, kind="rms"), dict(x=kt, weight=w[:1024], kind="rms")])
    kt = xt.clone()
    ops.adaln_multi([dict(x=qi, weight=w, kind="rms", out=qi), dict(x=kt, weight=w, kind="rms", out=kt)])
    assert torch.equal(qi, ops.adaln(xi, weight=w, kind="rms")) and torch.equal(kt, ops.adaln(xt, weight=w, kind="rms"))
    with pytest.raises(DitkError):  # one launch runs one norm kind
        ops.adaln_multi([dict(x=xi, weight=w), dict(x=xt, weight=w, kind="rms")])
    with pytest.raises(DitkError):  # at most four jobs
        ops.adaln_multi([dict(x=xt)] * 5)
    a, b = xt.clone(), xt.clone()
    with pytest.raises(ValueError):  # a job may not write another job's input (they run concurrently)
        ops.adaln_multi([dict(x=a, weight=w, kind="rms", out=b), dict(x=b, weight=w, kind="rms")])
    with pytest.raises(ValueError):  # nor share an output with it
        ops.adaln_multi([dict(x=a, weight=w, kind="rms", out=b), dict(x=xt, weight=w, kind="rms", out=b)])
    with pytest.raises(ValueError):  # an output of another row count
        ops.adaln(xi, weight=w, kind="rms", out=a)
    assert torch.equal(a, xt) and torch.equal(b, xt)


@pytest.mark.parametrize("per_head,Dh", [(True, 64), (True, 128), (False, 128)])
def test_qk_norm_multi_matches_single_calls(per_head, Dh):
    """One launch of RoPE-free QK-norm jobs (image and text, in place; a third
    out of place into column slices of another buffer) equals, bitwise, separate
    qk_norm_rope_() calls; jobs of another grouping are refused."""
    ops = _ops()
    from ditserve_amd._lib import DitkError
    D = 1536
    qkv_i = randn((1000, 3 * D), 96, 2.0).to(DEV, torch.bfloat16)
    qkv_t = randn((154, 3 * D), 97, 2.0).to(DEV, torch.bfloat16)
    n = D if not per_head else Dh
    wi = [(randn((n,), s, 0.1) + 1).repeat(D // n).to(DEV) for s in (98, 99)]
    wt = [(randn((n,), s, 0.1) + 1).repeat(D // n).to(DEV) for s in (100, 101)]
    ref_i, ref_t = qkv_i.clone(), qkv_t.clone()
    ops.qk_norm_rope_(ref_i[:, :D], ref_i[:, D:2 * D], *wi, Dh, per_head=per_head)
    ops.qk_norm_rope_(ref_t[:, :D], ref_t[:, D:2 * D], *wt, Dh, per_head=per_head)
    src = qkv_t.clone()
    buf = torch.zeros((154, 3 * D), dtype=torch.bfloat16, device=DEV)
    got = ops.qk_norm_multi([
        dict(q=qkv_i[:, :D], k=qkv_i[:, D:2 * D], wq=wi[0], wk=wi[1], head_dim=Dh, per_head=per_head),
        dict(q=qkv_t[:, :D], k=qkv_t[:, D:2 * D], wq=wt[0], wk=wt[1], head_dim=Dh, per_head=per_head),
        dict(q=src[:, :D], k=src[:, D:2 * D], wq=wt[0], wk=wt[1], head_dim=Dh, per_head=per_head,
             out=(buf[:, :D], buf[:, 2 * D:]))])
    assert torch.equal(qkv_i, ref_i) and torch.equal(qkv_t, ref_t)
    assert torch.equal(got[2][0], ref_t[:, :D]) and torch.equal(got[2][1], ref_t[:, D:2 * D])
    # zero-row jobs (empty views: NULL pointers) are skipped, alone or beside others
    e = torch.empty((0, 3 * D), dtype=torch.bfloat16, device=DEV)
    ops.qk_norm_rope_(e[:, :D], e[:, D:2 * D], *wt, Dh, per_head=per_head)
    before = qkv_t.clone()
    ops.qk_norm_multi([dict(q=e[:, :D], k=e[:, D:2 * D], wq=wt[0], wk=wt[1], head_dim=Dh, per_head=per_head),
                       dict(q=qkv_t[:, :D], k=qkv_t[:, D:2 * D], wq=wt[0], wk=wt[1], head_dim=Dh,
                            per_head=per_head)])
    again = before.clone()
    ops.qk_norm_rope_(again[:, :D], again[:, D:2 * D], *wt, Dh, per_head=per_head)
    assert torch.equal(qkv_t, again)
    assert torch.equal(buf[:, D:2 * D], torch.zeros_like(buf[:, D:2 * D])) and torch.equal(src[:, 2 * D:],
                                                                                            qkv_t[:, 2 * D:])
    other = dict(q=qkv_t[:, :D], k=qkv_t[:, D:2 * D], wq=wt[0], wk=wt[1], head_dim=64 if Dh == 128 else 128,
                 per_head=True)
    with pytest.raises(DitkError):
        ops.qk_norm_multi([dict(q=qkv_i[:, :D], k=qkv_i[:, D:2 * D], wq=wi[0], wk=wi[1], head_dim=Dh,
                                per_head=per_head), other])
    with pytest.raises(ValueError):  # one job's output over another job's q
        ops.qk_norm_multi([dict(q=qkv_t[:, :D], k=qkv_t[:, D:2 * D], wq=wt[0], wk=wt[1], head_dim=Dh,
                                per_head=per_head, out=(src[:, :D], src[:, 2 * D:])),
                           dict(q=src[:, :D], k=src[:, D:2 * D], wq=wt[0], wk=wt[1], head_dim=Dh, per_head=per_head)])


# --------------------------------------------------------------------------- attention
def _attn_case(cu_q, cu_k, H, Dh, seed, scale_in=1.0):
    q = bf(randn((cu_q[-1], H * Dh), seed, scale_in))
    k = bf(randn((cu_k[-1], H * Dh), seed + 1, scale_in))
    v = bf(randn((cu_k[-1], H * Dh), seed + 2))
    return q, k, v


def _attn_ref(q, k, v, cu_q, cu_k, H, Dh):
    return oc.varlen_attention(q.view(-1, H, Dh), k.view(-1, H, Dh), v.view(-1, H, Dh), cu_q, cu_k).flatten(1)


@pytest.mark.parametrize("Dh", [128, 64])
@pytest.mark.parametrize("lens", [[1], [63], [64], [65, 257], [300, 1, 129, 511], [1025]])
def test_self_attention_varlen(Dh, lens):
    ops = _ops()
    H = 3
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    q, k, v = _attn_case(cu, cu, H, Dh, 30, scale_in=2.0)
    out, lse = ops.flash_attn_varlen(q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16),
                                     v.to(DEV, torch.bfloat16), _seg(cu), _seg(cu), H, Dh, return_lse=True)
    ref = _attn_ref(q, k, v, cu, cu, H, Dh)
    assert_close(out.float().cpu(), ref, cos_min=0.9999, rel_max=1e-2, label=f"self {lens} Dh={Dh}")
    for m in range(len(lens)):
        s0, s1 = cu[m], cu[m + 1]
        qh, kh = q[s0:s1].view(-1, H, Dh).transpose(0, 1), k[s0:s1].view(-1, H, Dh).transpose(0, 1)
        ref_lse = torch.logsumexp((qh @ kh.transpose(1, 2)) / math.sqrt(Dh), dim=-1)
        assert torch.allclose(lse[:, s0:s1].cpu(), ref_lse, atol=2e-3, rtol=1e-4)


def test_attention_sharp_logits():
    """Large logits (|s| ~ 30): exercises the running max / rescale path."""
    ops = _ops()
    H, Dh, cu = 2, 128, [0, 700, 1500]
    q, k, v = _attn_case(cu, cu, H, Dh, 40, scale_in=4.0)
    out = ops.flash_attn_varlen(q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16), v.to(DEV, torch.bfloat16),
                                _seg(cu), _seg(cu), H, Dh).float().cpu()
    assert_close(out, _attn_ref(q, k, v, cu, cu, H, Dh), cos_min=0.999, rel_max=2e-2, label="sharp")


@pytest.mark.parametrize("Dh", [128, 64])
def test_attention_lse_merge_invariance(Dh):
    """Attention over a key range equals the LSE-weighted merge of attention over
    its two halves: O = (O1 e^lse1 + O2 e^lse2) / (e^lse1 + e^lse2), lse =
    log(e^lse1 + e^lse2) -- ties the kernel's output and its natural-log LSE
    together without restating the kernel's arithmetic.  Split at 700 (inside a
    key tile) of 1500 keys, two segments."""
    ops = _ops()
    H = 2
    cu_q, cu_k = [0, 300, 800], [0, 1500, 3000]
    q, k, v = _attn_case(cu_q, cu_k, H, Dh, 70, scale_in=2.0)
    qd, kd, vd = (t.to(DEV, torch.bfloat16) for t in (q, k, v))
    o, lse = ops.flash_attn_varlen(qd, kd, vd, _seg(cu_q), _seg(cu_k), H, Dh, return_lse=True)
    parts = []
    for lo, hi in ((0, 700), (700, 1500)):
        rows = torch.cat([torch.arange(b + lo, b + hi) for b in cu_k[:-1]]).to(DEV)
        ck = [0, hi - lo, 2 * (hi - lo)]
        parts.append(ops.flash_attn_varlen(qd, kd[rows].contiguous(), vd[rows].contiguous(), _seg(cu_q), _seg(ck), H,
                                           Dh, return_lse=True))
    (o1, l1), (o2, l2) = parts
    l1, l2 = l1.float().t().contiguous(), l2.float().t().contiguous()  # [T, H]
    m = torch.maximum(l1, l2)
    w1, w2 = torch.exp(l1 - m), torch.exp(l2 - m)
    o1, o2 = o1.float().view(-1, H, Dh), o2.float().view(-1, H, Dh)
    merged = (o1 * w1[..., None] + o2 * w2[..., None]) / (w1 + w2)[..., None]
    assert_close(o.float().view(-1, H, Dh).cpu(), merged.cpu(), cos_min=0.9999, rel_max=1e-2, label="merged O")
    assert torch.allclose(lse.float().t().cpu(), (m + torch.log(w1 + w2)).cpu(), atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("Dh", [128, 64])
def test_attention_rising_scores(Dh):
    """Scores rising by 0.3 per key (about 14 log2 units per 32 keys) for even query rows and
    falling for odd ones: the running max has to be raised in every half tile, inside the key
    loop and on each segment's last tile, while half the lanes of a wave keep their max."""
    ops = _ops()
    H, cu = 2, [0, 333, 1000, 1031]
    T = cu[-1]
    g = torch.Generator().manual_seed(80)
    u = torch.randn(H, Dh, generator=g)
    u = u / u.norm(dim=1, keepdim=True)
    sign = torch.where(torch.arange(T) % 2 == 0, 1.0, -1.0)
    q = (math.sqrt(Dh) * sign[:, None, None] * u[None]).expand(T, H, Dh)
    pos = torch.cat([torch.arange(cu[m + 1] - cu[m], dtype=torch.float32) for m in range(len(cu) - 1)])
    k = 0.3 * pos[:, None, None] * u[None] + 0.1 * torch.randn(T, H, Dh, generator=g)
    v = torch.randn(T, H, Dh, generator=g)
    q, k, v = (bf(t.reshape(T, H * Dh)) for t in (q, k, v))
    seg = _seg(cu)
    out = ops.flash_attn_varlen(q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16), v.to(DEV, torch.bfloat16),
                                seg, seg, H, Dh).float().cpu()
    assert_close(out, _attn_ref(q, k, v, cu, cu, H, Dh), cos_min=0.9999, rel_max=1e-2, label=f"rising Dh={Dh}")


@pytest.mark.parametrize("Dh", [128, 64])
@pytest.mark.parametrize("case", ["random", "rising"])
@pytest.mark.parametrize("lens", [[1], [64, 65], [300, 1, 129, 511], [1025]])
def test_attention_q_prescaled(Dh, case, lens):
    """q already multiplied by softmax_scale*log2(e): the kernel starts its score
    accumulators at -max and must move them, and the next tile's already computed scores,
    whenever the max rises (rising scores force that in every tile).  Reference: the oracle
    on the same bf16 q' rescaled back by ln 2 * sqrt(Dh) in fp32, so that its
    softmax(q.k / sqrt(Dh)) equals 2^(q'.k)."""
    ops = _ops()
    H = 3
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    T = cu[-1]
    if case == "random":
        q, k, v = _attn_case(cu, cu, H, Dh, 90, scale_in=2.0)
    else:
        g = torch.Generator().manual_seed(91)
        u = torch.randn(H, Dh, generator=g)
        u = u / u.norm(dim=1, keepdim=True)
        sign = torch.where(torch.arange(T) % 2 == 0, 1.0, -1.0)
        q = (math.sqrt(Dh) * sign[:, None, None] * u[None]).expand(T, H, Dh)
        pos = torch.cat([torch.arange(cu[m + 1] - cu[m], dtype=torch.float32) for m in range(len(cu) - 1)])
        k = 0.3 * pos[:, None, None] * u[None] + 0.1 * torch.randn(T, H, Dh, generator=g)
        v = torch.randn(T, H, Dh, generator=g)
        q, k, v = (bf(t.reshape(T, H * Dh)) for t in (q, k, v))
    qp = bf(q * (ops.LOG2E / math.sqrt(Dh)))  # what a QK-norm with the folded weight emits
    seg = _seg(cu)
    out, lse = ops.flash_attn_varlen(qp.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16),
                                     v.to(DEV, torch.bfloat16), seg, seg, H, Dh, return_lse=True, q_prescaled=True)
    q_ref = qp * (math.log(2.0) * math.sqrt(Dh))
    ref = _attn_ref(q_ref, k, v, cu, cu, H, Dh)
    assert_close(out.float().cpu(), ref, cos_min=0.9999, rel_max=1e-2, label=f"prescaled {case} {lens}")
    for m in range(len(lens)):
        s0, s1 = cu[m], cu[m + 1]
        qh, kh = q_ref[s0:s1].view(-1, H, Dh).transpose(0, 1), k[s0:s1].view(-1, H, Dh).transpose(0, 1)
        ref_lse = torch.logsumexp((qh @ kh.transpose(1, 2)) / math.sqrt(Dh), dim=-1)
        assert torch.allclose(lse[:, s0:s1].cpu(), ref_lse, atol=2e-3, rtol=1e-4)


@pytest.mark.parametrize("Dh", [128, 64])
@pytest.mark.parametrize("pre", [False, True])
@pytest.mark.parametrize("cu_k", [[0, 300, 377, 377], [0, 40, 104, 104]])
def test_attention_query_tile_passes_bitwise(Dh, pre, cu_k):
    """Short key ranges over many query tiles run several query tiles per workgroup, the
    next tile's loads issued under the current one's last key tile.  With 16 heads the call
    takes that path; one head at a time (too few tiles to fill the GPU that way) runs one
    tile per workgroup: the outputs must be bitwise equal.  Segments: 65 query tiles (the
    last work item one pass short) over 5 key tiles (or one partial tile), 64 over 2 (or one
    full tile), and 2 over none; sampled rows are checked against the oracle."""
    ops = _ops()
    H = 16
    cu_q = [0, 16484, 32768, 33280]
    g = torch.Generator(device=DEV).manual_seed(98)
    q = torch.randn((cu_q[-1], H * Dh), generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn((cu_k[-1], H * Dh), generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn((cu_k[-1], H * Dh), generator=g, device=DEV).to(torch.bfloat16)
    if pre:
        q = (q.float() * (ops.LOG2E / math.sqrt(Dh))).to(torch.bfloat16)
    sq, sk = _seg(cu_q), _seg(cu_k)
    full, lse = ops.flash_attn_varlen(q, k, v, sq, sk, H, Dh, return_lse=True, q_prescaled=pre)
    for h in range(H):
        cols = slice(h * Dh, (h + 1) * Dh)
        one, lse1 = ops.flash_attn_varlen(q[:, cols], k[:, cols], v[:, cols], sq, sk, 1, Dh, return_lse=True,
                                          q_prescaled=pre)
        assert torch.equal(one, full[:, cols]), f"head {h}"
        assert torch.equal(lse1[0], lse[h]), f"lse head {h}"
    rows = torch.tensor([0, 255, 256, 16383, 16483, 16484, 16740, 32767], device=DEV)
    qs = q[rows].float().cpu()
    q_ref = qs * (math.log(2.0) * math.sqrt(Dh)) if pre else qs
    for i, r in enumerate(rows.tolist()):
        m = 0 if r < cu_q[1] else 1
        ref = _attn_ref(q_ref[i:i + 1], k[cu_k[m]:cu_k[m + 1]].float().cpu(), v[cu_k[m]:cu_k[m + 1]].float().cpu(),
                        [0, 1], [0, cu_k[m + 1] - cu_k[m]], H, Dh)
        assert_close(full[r:r + 1].float().cpu(), ref, cos_min=0.999, rel_max=1e-2, label=f"row {r}")
    assert torch.equal(full[32768:], torch.zeros_like(full[32768:]))
    assert bool(torch.all(lse[:, 32768:] == -math.inf))


def test_empty_inputs_are_no_ops():
    """Zero-row GEMM inputs and zero-query or zero-key attention calls (empty
    tensors: NULL pointers) launch nothing and return empty or zero-filled outputs."""
    ops = _ops()
    w, b = torch.zeros((64, 64), dtype=torch.bfloat16, device=DEV), torch.zeros(64, device=DEV)
    x0 = torch.empty((0, 64), dtype=torch.bfloat16, device=DEV)
    assert ops.linear(x0, w, b).shape == (0, 64)
    assert ops.linear(x0, w, b, "res", residual=torch.empty((0, 64), dtype=torch.bfloat16, device=DEV)).shape == (0, 64)
    q0 = torch.empty((0, 128), dtype=torch.bfloat16, device=DEV)
    kv = randn((40, 128), 3).to(DEV, torch.bfloat16)
    assert ops.flash_attn_varlen(q0, kv, kv, _seg([0, 0]), _seg([0, 40]), 1, 128).shape == (0, 128)
    q = randn((40, 128), 4).to(DEV, torch.bfloat16)
    k0 = torch.empty((0, 128), dtype=torch.bfloat16, device=DEV)
    out, lse = ops.flash_attn_varlen(q, k0, k0, _seg([0, 40]), _seg([0, 0]), 1, 128, return_lse=True)
    assert torch.equal(out, torch.zeros_like(out)) and bool(torch.isneginf(lse).all())
    torch.cuda.synchronize()


@pytest.mark.parametrize("Dh", [128, 64])
@pytest.mark.parametrize("pre", [False, True])
def test_attention_segments_without_keys(Dh, pre):
    """A segment with no keys (first and last here, the last one starting at the end of
    K) attends to nothing: zero output rows and lse = -inf; the others are unaffected."""
    ops = _ops()
    H = 2
    cu_q, cu_k = [0, 100, 300, 301], [0, 0, 130, 130]
    q, k, v = _attn_case(cu_q, cu_k, H, Dh, 97)
    qd = bf(q * (ops.LOG2E / math.sqrt(Dh))) if pre else q
    out, lse = ops.flash_attn_varlen(qd.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16),
                                     v.to(DEV, torch.bfloat16), _seg(cu_q), _seg(cu_k), H, Dh, return_lse=True,
                                     q_prescaled=pre)
    out, lse = out.float().cpu(), lse.cpu()
    for s0, s1 in ((0, 100), (300, 301)):
        assert torch.equal(out[s0:s1], torch.zeros_like(out[s0:s1]))
        assert bool(torch.all(lse[:, s0:s1] == -math.inf))
    q_ref = qd * (math.log(2.0) * math.sqrt(Dh)) if pre else q
    ref = _attn_ref(q_ref[100:300], k, v, [0, 200], [0, 130], H, Dh)
    assert_close(out[100:300], ref, cos_min=0.9999, rel_max=1e-2, label=f"no-keys neighbours Dh={Dh} pre={pre}")


@pytest.mark.parametrize("Dh", [128, 64])
def test_cross_attention_text_blocks(Dh):
    ops = _ops()
    H = 4
    cu_q, cu_k = [0, 900, 1000, 1777], [0, 512, 1024, 1536]
    q, k, v = _attn_case(cu_q, cu_k, H, Dh, 50)
    k[512 + 77:1024] = 0  # zero-padded text rows still attend
    v[512 + 77:1024] = 0
    out = ops.flash_attn_varlen(q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16), v.to(DEV, torch.bfloat16),
                                _seg(cu_q), _seg(cu_k), H, Dh).float().cpu()
    assert_close(out, _attn_ref(q, k, v, cu_q, cu_k, H, Dh), cos_min=0.9999, rel_max=1e-2, label="cross")


def test_attention_packed_equals_solo_bitwise():
    ops = _ops()
    H, Dh = 2, 128
    lens = [300, 1, 513, 64]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    q, k, v = (t.to(DEV, torch.bfloat16) for t in _attn_case(cu, cu, H, Dh, 60))
    packed = ops.flash_attn_varlen(q, k, v, _seg(cu), _seg(cu), H, Dh)
    for m in range(len(lens)):
        s0, s1 = cu[m], cu[m + 1]
        solo = ops.flash_attn_varlen(q[s0:s1].contiguous(), k[s0:s1].contiguous(), v[s0:s1].contiguous(),
                                     _seg([0, s1 - s0]), _seg([0, s1 - s0]), H, Dh)
        assert torch.equal(packed[s0:s1], solo), f"segment {m}"


def test_attention_full_length_sampled_rows():
    """S = 32760 (one Wan2.1 480p request): every K/V tile of the full sequence, checked
    on 192 sampled query rows against the oracle."""
    ops = _ops()
    H, Dh, S = 2, 128, 32760
    q, k, v = _attn_case([0, S], [0, S], H, Dh, 70)
    out = ops.flash_attn_varlen(q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16), v.to(DEV, torch.bfloat16),
                                _seg([0, S]), _seg([0, S]), H, Dh).float().cpu()
    rows = torch.cat([torch.arange(0, 64), torch.randint(64, S - 64, (64,), generator=torch.Generator().manual_seed(1)),
                      torch.arange(S - 64, S)])
    qs = q[rows].view(-1, H, Dh).transpose(0, 1)
    ref = oc.sdpa(qs, k.view(S, H, Dh).transpose(0, 1), v.view(S, H, Dh).transpose(0, 1)).transpose(0, 1).flatten(1)
    assert_close(out[rows], ref, cos_min=0.9999, rel_max=1e-2, label="S=32760 sampled")


# --------------------------------------------------------------------------- glue
def test_patchify_unpatchify_roundtrip_and_oracle():
    ops = _ops()
    C, F, H, W = 16, 3, 6, 10
    lat = bf(randn((C, F, H, W), 80))
    p = ops.patchify(lat.to(DEV, torch.bfloat16), (1, 2, 2)).float().cpu()
    ref = lat.reshape(C, F, 1, H // 2, 2, W // 2, 2).permute(1, 3, 5, 0, 2, 4, 6).reshape(F * (H // 2) * (W // 2), -1)
    assert torch.equal(p, ref)
    # unpatchify with the (i, j, l, c) feature order of proj_out
    x = bf(randn((F * (H // 2) * (W // 2), 4 * C), 81))
    u = ops.unpatchify(x.to(DEV, torch.bfloat16), (F, H // 2, W // 2), (1, 2, 2), C).cpu()
    ref_u = x.reshape(F, H // 2, W // 2, 1, 2, 2, C).permute(6, 0, 3, 1, 4, 2, 5).reshape(C, F, H, W)
    assert torch.equal(u, ref_u)


def test_timestep_embedding_and_cfg():
    ops = _ops()
    t = torch.tensor([0.0, 1.0, 500.0, 999.0])
    e = ops.timestep_embedding(t.to(DEV), 256).float().cpu()
    assert_close(e, oc.timestep_embedding(t, 256), cos_min=0.99999, rel_max=5e-3, label="temb")
    c, u = randn((1000,), 82), randn((1000,), 83)
    out = ops.cfg_combine(c.to(DEV), u.to(DEV), 5.0).cpu()
    assert torch.allclose(out, u + 5.0 * (c - u), atol=1e-5)


@pytest.mark.parametrize("img,txt", [([300, 4096], [77, 333]), ([64, 0, 130], [0, 40, 333]), ([1], [63]),
                                     ([0, 100], [50, 0])])
def test_joint_attention_two_sources_bitwise(img, txt):
    """Joint attention read straight from the image and text buffers (and V transposed
    from them) is bitwise the gather -> pre-scaled flash -> scatter path, including
    segments without text or without image rows and tiles across the image/text seam."""
    ops = _ops()
    H, Dh, W = 4, 64, 3 * 4 * 64
    cu_i, cu_t = [0], [0]
    for a, b in zip(img, txt):
        cu_i.append(cu_i[-1] + a)
        cu_t.append(cu_t[-1] + b)
    cu_j = [a + b for a, b in zip(cu_i, cu_t)]
    g = torch.Generator(device=DEV).manual_seed(95)
    qkv_i = (torch.randn((cu_i[-1], W), generator=g, device=DEV) * 0.3).to(torch.bfloat16)
    qkv_t = (torch.randn((cu_t[-1], W), generator=g, device=DEV) * 0.3).to(torch.bfloat16)
    si, st, sj = _seg(cu_i), _seg(cu_t), _seg(cu_j)
    D = H * Dh
    joint = ops.joint_gather(qkv_i, qkv_t, si, st)
    vt_ref = ops.transpose_v(joint[:, 2 * D:], H, Dh, sj)
    ref = ops.flash_attn_varlen(joint[:, :D], joint[:, D:2 * D], None, sj, sj, H, Dh, vt=vt_ref, q_prescaled=True)
    ref_i = torch.empty((cu_i[-1], D), dtype=torch.bfloat16, device=DEV)
    ref_t = torch.empty((cu_t[-1], D), dtype=torch.bfloat16, device=DEV)
    ops.joint_scatter(ref, ref_i, ref_t, si, st)
    vt = ops.transpose_v_joint(qkv_i[:, 2 * D:], qkv_t[:, 2 * D:], H, Dh, si, st, sj)
    used = sum(-(-(b - a) // 64) * 64 for a, b in zip(cu_j, cu_j[1:]))  # written columns; the rest is slack
    assert torch.equal(vt[:, :, :used], vt_ref[:, :, :used])
    o_i, o_t = ops.joint_attention_q_prescaled(qkv_i[:, :D], qkv_t[:, :D], qkv_i[:, D:2 * D], qkv_t[:, D:2 * D],
                                               vt, si, st, sj, H, Dh)
    assert torch.equal(o_i, ref_i) and torch.equal(o_t, ref_t)


def test_joint_attention_rejects_inconsistent_tables():
    ops = _ops()
    x = torch.zeros((64, 256), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="cu_joint"):
        ops.transpose_v_joint(x[:32], x[:32], 4, 64, _seg([0, 32]), _seg([0, 32]), _seg([0, 60]))


def test_joint_gather_scatter_roundtrip():
    ops = _ops()
    img_counts, txt_counts = [40, 7, 100], [33, 33, 33]
    si, st = _seg([0, 40, 47, 147]), _seg([0, 33, 66, 99])
    img = randn((147, 128), 84).to(DEV, torch.bfloat16)
    txt = randn((99, 128), 85).to(DEV, torch.bfloat16)
    joint = ops.joint_gather(img, txt, si, st)
    from ditserve_amd.packing import joint_layout
    lay = joint_layout(img_counts, txt_counts)
    assert torch.equal(joint[torch.tensor(lay["img_in_joint"], device=DEV)], img)
    assert torch.equal(joint[torch.tensor(lay["txt_in_joint"], device=DEV)], txt)
    img2, txt2 = torch.zeros_like(img), torch.zeros_like(txt)
    ops.joint_scatter(joint, img2, txt2, si, st)
    assert torch.equal(img2, img) and torch.equal(txt2, txt)


@pytest.mark.parametrize("hd", [64, 128])
def test_transpose_v_layout(hd):
    """Vt[h, d, pk_m + j] = V[cu[m] + j, h * hd + d] for the rows of segment m,
    zero up to its 64-padded end (pk_m = the padded lengths of the segments
    before it); V is a column slice of a fused QKV row (ragged and empty
    segments, one key, a tile boundary)."""
    ops = _ops()
    H, cu = 3, [0, 1, 130, 130, 333, 397]
    T = cu[-1]
    qkv = randn((T, 3 * H * hd), 90).to(DEV, torch.bfloat16)
    v = qkv[:, 2 * H * hd:]
    vt = ops.transpose_v(v, H, hd, _seg(cu)).cpu()
    vc = v.cpu()
    pk = 0
    for m in range(len(cu) - 1):
        n = cu[m + 1] - cu[m]
        padded = (n + 63) // 64 * 64
        want = torch.zeros((H, hd, padded), dtype=torch.bfloat16)
        want[:, :, :n] = vc[cu[m]:cu[m + 1]].reshape(n, H, hd).permute(1, 2, 0)
        assert torch.equal(vt[:, :, pk:pk + padded], want), (hd, m)
        pk += padded


def test_invalid_arguments_raise_before_launch():
    ops = _ops()
    from ditserve_amd._lib import DitkError
    x = torch.zeros((10, 96), dtype=torch.bfloat16, device=DEV)
    with pytest.raises((ValueError, DitkError)):
        ops.flash_attn_varlen(x, x, x, _seg([0, 10]), _seg([0, 10]), 1, 96)  # head_dim 96 unsupported
    with pytest.raises(ValueError):
        ops.linear(x, torch.zeros((8, 64), dtype=torch.bfloat16, device=DEV))  # K mismatch
    q = torch.zeros((4, 128), dtype=torch.bfloat16, device=DEV)
    w = torch.ones((128,), dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError):  # out-of-place output of another shape
        ops.qk_norm_rope_(q, q.clone(), w, w, 64, out=(torch.empty((4, 64), dtype=torch.bfloat16, device=DEV), q.clone()))
    big = torch.zeros((4, 136), dtype=torch.bfloat16, device=DEV)
    with pytest.raises((ValueError, DitkError)):  # output rows not 16-byte aligned (4-element column offset)
        ops.qk_norm_rope_(q, q.clone(), w, w, 64, out=(big[:, 4:132], q.clone()))
    assert torch.equal(q, torch.zeros_like(q))
    # caller-supplied outputs and operands of the wrong size are refused before any launch
    v = torch.zeros((10, 256), dtype=torch.bfloat16, device=DEV)
    seg = _seg([0, 4, 10])
    with pytest.raises(ValueError):  # v narrower than heads * head_dim
        ops.transpose_v(v, 3, 128, seg)
    with pytest.raises(ValueError):  # Vt buffer too small
        ops.transpose_v(v, 2, 128, seg, out=torch.empty((2, 128, 64), dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError):  # table of another token count
        ops.transpose_v(v, 2, 128, _seg([0, 4, 9]))
    with pytest.raises(ValueError):  # attention output of too few rows
        ops.flash_attn_varlen(v, v, v, seg, seg, 2, 128, out=torch.empty((9, 256), dtype=torch.bfloat16, device=DEV))
    img, txt = torch.zeros((10, 64), dtype=torch.bfloat16, device=DEV), torch.zeros((6, 64), dtype=torch.bfloat16,
                                                                                   device=DEV)
    si, st = _seg([0, 4, 10]), _seg([0, 3, 6])
    with pytest.raises(ValueError):  # text rows of another width
        ops.joint_gather(img, torch.zeros((6, 128), dtype=torch.bfloat16, device=DEV), si, st)
    with pytest.raises(ValueError):  # joint buffer of too few rows
        ops.joint_gather(img, txt, si, st, out=torch.empty((15, 64), dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError):  # scatter source of too few rows
        ops.joint_scatter(torch.empty((15, 64), dtype=torch.bfloat16, device=DEV), img, txt, si, st)
    with pytest.raises(ValueError):  # joint attention output of too few rows
        vtj = torch.zeros((1, 64, ops.vt_columns(16, 2)), dtype=torch.bfloat16, device=DEV)
        ops.joint_attention_q_prescaled(img, txt, img, txt, vtj, si, st, _seg([0, 7, 16]), 1, 64, out_img=img[:9])
    with pytest.raises(ValueError):  # rows that are not the grid's tokens
        ops.unpatchify(torch.zeros((11, 64), dtype=torch.bfloat16, device=DEV), (1, 2, 5), (1, 2, 2), 16)
    with pytest.raises(ValueError):  # CFG branches of different sizes
        ops.cfg_combine(torch.zeros(8, device=DEV), torch.zeros(6, device=DEV), 5.0)
    with pytest.raises(DitkError):  # rows wider than the row kernels hold in registers (6144)
        ops.adaln(torch.zeros((4, 6152), dtype=torch.bfloat16, device=DEV))
    xr = torch.zeros((4, 64), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):  # a strided weight view (the kernel reads a contiguous vector)
        ops.adaln(xr, weight=torch.ones(128, device=DEV)[::2])
    with pytest.raises(ValueError):  # scale without shift
        ops.adaln(xr, scale=torch.zeros((1, 64), device=DEV), segments=_seg([0, 4]))
    from ditserve_amd.wan import rope_tables
    cos_t, sin_t = rope_tables(128, 16, 10000.0, DEV)
    with pytest.raises(ValueError):  # a grid longer than the 16-position RoPE tables
        ops.Rope(cos_t, sin_t, [(2, 20, 1)], _seg([0, 40]), 22, 21)
    with pytest.raises(ValueError):  # tables for head_dim 128 on head_dim-64 rows
        q64 = torch.zeros((40, 128), dtype=torch.bfloat16, device=DEV)
        ops.qk_norm_rope_(q64, q64.clone(), torch.ones(128, device=DEV), torch.ones(128, device=DEV), 64,
                          rope=ops.Rope(cos_t, sin_t, [(2, 4, 5)], _seg([0, 40]), 22, 21))
    with pytest.raises(ValueError):  # a strided bias
        ops.linear(xr, torch.zeros((64, 64), dtype=torch.bfloat16, device=DEV), torch.zeros(128, device=DEV)[::2])
    torch.cuda.synchronize()
