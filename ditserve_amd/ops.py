"""Tensor-level wrappers over the ditk C ABI.

Every op validates device, dtype, layout and shape on the host (raising
ValueError before any launch, as the reference's ``Spec.rejects`` does at
workers/xfuser/core/attention/spec.py:244-246), allocates outputs with
``torch.empty`` when none is given, and launches on the caller's current
stream without synchronising.  There is no CPU or PyTorch fallback.
"""
import ctypes
import math

import torch

from . import _lib

EPILOGUES = {"bias": 0, "gelu": 1, "gate_res": 2, "res": 3, "f32": 4, "silu": 5}
_BF16 = torch.bfloat16


def _stream():
    return ctypes_stream(torch.cuda.current_stream())


def ctypes_stream(stream):
    return _lib.c_void_p(stream.cuda_stream)


def _ptr(t):
    return _lib.c_void_p(t.data_ptr()) if t is not None else None


def _check(t, name, dtype=None, dims=None):
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a cuda (HIP) device, got {t.device}")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if dims is not None and t.dim() != dims:
        raise ValueError(f"{name} must be {dims}-D, got shape {tuple(t.shape)}")


def to_device(data, dtype, device):
    """Small host table -> device tensor without stalling the host: the values go
    through pinned memory and a non-blocking copy on the current stream (a
    pageable copy would wait for all work already queued on the stream)."""
    host = torch.tensor(data, dtype=dtype)
    if torch.device(device).type != "cuda":
        return host.to(device)
    return host.pin_memory().to(device, non_blocking=True)


def _vec(t, name, n):
    """An fp32 per-feature vector (norm weight, bias): 1-D, n long, unit stride (the
    kernels read it as a contiguous array)."""
    _check(t, name, torch.float32, 1)
    if t.shape[0] != n or (n > 1 and t.stride(0) != 1):
        raise ValueError(f"{name} must be a contiguous [{n}] vector, got shape {tuple(t.shape)} "
                         f"stride {t.stride()}")


def _rows(t, name):
    """2-D row-major view requirements: unit column stride, 16-byte aligned rows."""
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D tensor with unit column stride, got strides {t.stride()}")
    if t.stride(0) % 8 or t.data_ptr() % 16:
        raise ValueError(f"{name} rows must be 16-byte aligned (leading dim % 8 == 0)")
    return t.stride(0)


class Segments:
    """Packed-batch segment table: host list of offsets + device int32 copy.

    ``cu`` follows build_cu_seqlens (workers/ditserve/models/sd35_batch.py:135-145):
    [0, n0, n0+n1, ...]."""

    def __init__(self, cu, device):
        self.cu = [int(x) for x in cu]
        if not self.cu or self.cu[0] != 0 or any(b < a for a, b in zip(self.cu, self.cu[1:])):
            raise ValueError(f"cu_seqlens must start at 0 and be nondecreasing, got {self.cu}")
        self.dev = to_device(self.cu, torch.int32, device)
        self._nseg, self._total = len(self.cu) - 1, self.cu[-1]

    @classmethod
    def from_device(cls, cu_dev, total):
        """Wrap a caller's device int32 cu_seqlens tensor without reading it back
        (no host sync).  A small kernel first copies it into a table of its own,
        clamped so that every segment lies inside [0, total); a table that was not
        valid (cu[0] != 0, a decrease, cu[-1] != total) sets the device's sticky
        status, which the next call made after that kernel has finished raises
        (table_status(...).poll()), or check_tables() raises after a sync."""
        if cu_dev.dtype != torch.int32 or cu_dev.dim() != 1 or cu_dev.numel() < 2 or cu_dev.device.type != "cuda":
            raise ValueError("cu_seqlens must be a 1-D int32 cuda tensor with at least 2 entries")
        status = table_status(cu_dev.device)
        status.poll()
        obj = cls.__new__(cls)
        obj.cu = None
        obj.dev = torch.empty_like(cu_dev, memory_format=torch.contiguous_format)
        obj._nseg, obj._total = cu_dev.numel() - 1, int(total)
        _lib.call("ditk_check_cu_seqlens", _ptr(cu_dev.contiguous()), obj._nseg, obj._total, _ptr(obj.dev),
                  _ptr(status.dev), _stream())
        status.queue_read()
        return obj

    @classmethod
    def uniform(cls, count, length, device):
        """[0, length, 2 length, ...] for `count` equal segments, cached per
        (device, count, length): after the first call no host upload happens.
        The cached table is uploaded synchronously once, so any stream may read it."""
        key = (torch.device(device), int(count), int(length))
        seg = _UNIFORM.get(key)
        if seg is None:
            obj = cls.__new__(cls)
            obj.cu = [i * int(length) for i in range(int(count) + 1)]
            obj.dev = torch.tensor(obj.cu, dtype=torch.int32).to(device)
            torch.cuda.current_stream(obj.dev.device).synchronize()
            obj._nseg, obj._total = int(count), obj.cu[-1]
            if len(_UNIFORM) >= 64:
                _UNIFORM.clear()
            seg = _UNIFORM[key] = obj
        return seg

    @property
    def nseg(self):
        return self._nseg

    @property
    def total(self):
        return self._total

    @property
    def max_len(self):
        return max(b - a for a, b in zip(self.cu, self.cu[1:]))

    def lengths(self):
        return [b - a for a, b in zip(self.cu, self.cu[1:])]

    def device_tensors(self):
        return (self.dev,)

    def record_stream(self, stream):
        """Mark the device table as in use by ``stream`` (for packets consumed on a
        side stream, as the reference's interleaved executor does)."""
        self.dev.record_stream(stream)


_UNIFORM = {}


class TableStatus:
    """Sticky per-device flag of ditk_check_cu_seqlens.  After each check a copy of
    the flag goes to pinned host memory without blocking; poll() looks at it only
    once that copy has completed (an event query, never a wait) and raises if a
    table was invalid.  check() waits for the device and raises likewise."""

    def __init__(self, device):
        self.dev = torch.zeros(1, dtype=torch.int32, device=device)
        self.host = torch.zeros(1, dtype=torch.int32).pin_memory()
        self.event = None

    def queue_read(self):
        self.host.copy_(self.dev, non_blocking=True)
        self.event = torch.cuda.Event()
        self.event.record()

    def _raise_if_set(self):
        if int(self.host[0]) != 0:
            self.host.zero_()
            self.dev.zero_()
            self.event = None
            raise _lib.DitkError("an invalid cu_seqlens table reached the attention kernels (cu[0] != 0, "
                                 "decreasing, or its last entry != the packed token count); it was clamped "
                                 "into bounds, so those outputs are not attention over the intended segments")

    def poll(self):
        if self.event is not None and self.event.query():
            self._raise_if_set()

    def check(self):
        torch.cuda.synchronize(self.dev.device)
        self.host.copy_(self.dev)
        self._raise_if_set()


_STATUS = {}


def table_status(device):
    device = torch.device(device)
    if device.index is None:
        device = torch.device(device.type, torch.cuda.current_device())
    st = _STATUS.get(device)
    if st is None:
        st = _STATUS[device] = TableStatus(device)
    return st


def check_tables(device=None):
    """Wait for `device` (default: the current one) and raise DitkError if a
    caller's cu_seqlens table checked since the last report was invalid."""
    table_status(device if device is not None else torch.device("cuda")).check()


# ---------------------------------------------------------------------------
# normalisation
# ---------------------------------------------------------------------------

def adaln(x, shift=None, scale=None, segments=None, weight=None, bias=None, eps=1e-6, kind="ln", out=None):
    """y = norm(x)[*w + b][*(1 + scale[seg]) + shift[seg]] -> bf16.

    x [T, D] bf16; shift/scale fp32 views [nseg, D] (row stride may exceed D);
    weight/bias fp32 [D]; kind "ln" (LayerNorm) or "rms" (RMSNorm)."""
    out, job = _adaln_job(x, shift, scale, segments, weight, bias, eps, kind, out)
    _lib.call("ditk_adaln", job.x, job.ldx, job.y, job.ldy, job.T, job.D, job.cu_seqlens, job.nseg, job.shift,
              job.scale, job.mod_stride, job.weight, job.bias, job.eps, job.norm_kind, _stream())
    return out


def adaln_multi(jobs):
    """Several adaln() calls (dicts of its keyword arguments, x required) in one
    launch: 1 to 4 jobs of one kind and one ceil(D / 512).  Returns the outputs;
    each is bitwise what adaln() returns for its job.  The jobs run concurrently:
    a job's output may be its own x (in place) but may not overlap another
    job's tensors."""
    built = [_adaln_job(**j) for j in jobs]
    _disjoint_jobs("adaln_multi", [((b[0],), tuple(j.get(k) for k in ("x", "shift", "scale", "weight", "bias")))
                                   for j, b in zip(jobs, built)])
    arr = (_lib.AdalnJob * len(built))(*[b[1] for b in built])
    _lib.call("ditk_adaln_multi", arr, len(built), _stream())
    return [b[0] for b in built]


def _adaln_job(x, shift=None, scale=None, segments=None, weight=None, bias=None, eps=1e-6, kind="ln", out=None):
    """Checks one adaln() call; returns (out, its ditk_adaln_job)."""
    _check(x, "x", _BF16, 2)
    T, D = x.shape
    ldx = _rows(x, "x")
    if out is None:
        out = torch.empty((T, D), dtype=_BF16, device=x.device)
    _check(out, "out", _BF16, 2)
    if out.shape != (T, D):
        raise ValueError(f"out must be [{T}, {D}], got {tuple(out.shape)}")
    ldy = _rows(out, "out")
    mod_stride = 0
    cu = None
    nseg = 0
    if (shift is None) != (scale is None):
        raise ValueError("shift and scale go together")
    if shift is not None:
        _check(shift, "shift", torch.float32, 2)
        _check(scale, "scale", torch.float32, 2)
        if segments is None:
            raise ValueError("modulation requires segments")
        if shift.shape != (segments.nseg, D) or scale.shape != (segments.nseg, D):
            raise ValueError(f"shift/scale must be [{segments.nseg}, {D}]")
        if shift.stride(1) != 1 or scale.stride(0) != shift.stride(0):
            raise ValueError("shift/scale must share a row stride with unit column stride")
        if segments.total != T:
            raise ValueError(f"segments cover {segments.total} tokens, x has {T}")
        mod_stride = shift.stride(0)
        cu, nseg = segments.dev, segments.nseg
    for t, n in ((weight, "weight"), (bias, "bias")):
        if t is not None:
            _vec(t, n, D)
    if kind not in ("ln", "rms"):
        raise ValueError(f"kind must be 'ln' or 'rms', got {kind!r}")
    job = _lib.AdalnJob(_ptr(x), ldx, _ptr(out), ldy, _ptr(cu), _ptr(shift), _ptr(scale), mod_stride, _ptr(weight),
                        _ptr(bias), T, D, nseg, {"ln": 0, "rms": 1}[kind], float(eps))
    return out, job


def modulation(table, proj):
    """fp32 [nseg, k, D] = table [k, D] + proj [nseg, k, D]  (the reference's
    ``scale_shift_table + temb.float()``, workers/ditserve/models/wan/block.py:276-280)."""
    _check(table, "table", torch.float32)
    _check(proj, "proj", torch.float32)
    table = table.reshape(-1).contiguous()
    proj = proj.contiguous()
    kd = table.numel()
    if proj.numel() % kd:
        raise ValueError("proj size is not a multiple of the table size")
    nseg = proj.numel() // kd
    out = torch.empty_like(proj)
    _lib.call("ditk_modulation", _ptr(table), _ptr(proj), _ptr(out), nseg, kd, _stream())
    return out


class Rope:
    """3D RoPE description for a packed batch: per-axis cos/sin tables
    [max_pos, head_dim/2] fp32 (float64-built), per-segment (F', H', W') grids."""

    def __init__(self, cos_tab, sin_tab, grids, segments, t_pairs, h_pairs):
        for t, n in ((cos_tab, "cos table"), (sin_tab, "sin table")):
            _check(t, n, torch.float32, 2)
            if not t.is_contiguous() or t.shape != cos_tab.shape:
                raise ValueError("the cos and sin tables must be contiguous [max_pos, head_dim / 2] fp32")
        for g in grids:
            if max(g) > cos_tab.shape[0]:
                raise ValueError(f"grid {tuple(g)} reaches past the {cos_tab.shape[0]}-position RoPE tables")
        self.cos, self.sin = cos_tab, sin_tab
        self.grids = to_device([list(map(int, g)) for g in grids], torch.int32, cos_tab.device).reshape(-1)
        self.segments = segments
        self.t_pairs, self.h_pairs = int(t_pairs), int(h_pairs)
        if len(grids) != segments.nseg:
            raise ValueError("one grid per segment required")
        for g, n in zip(grids, segments.lengths()):
            if g[0] * g[1] * g[2] != n:
                raise ValueError(f"grid {g} does not cover segment of {n} tokens")

    def __iter__(self):
        """The tensors a packet codec carries for the rotation: the two angle
        tables.  The per-token rotation is rebuilt from them and the packet's
        per-request grids."""
        return iter((self.cos, self.sin))

    def __len__(self):
        return 2

    def device_tensors(self):
        return (self.cos, self.sin, self.grids, *self.segments.device_tensors())

    def record_stream(self, stream):
        for t in self.device_tensors():
            t.record_stream(stream)


def qk_norm_multi(jobs):
    """Several RoPE-free qk_norm_rope_() calls in one launch: jobs are dicts with
    q, k, wq, wk, head_dim and optionally eps, per_head, out (1 to 4 jobs of one
    ceil(D / 512), head_dim and per_head).  Each job's result is bitwise what
    qk_norm_rope_() gives it; returns the (q, k) pairs written.  The jobs run
    concurrently: a job may write in place, but its outputs may not overlap
    another job's tensors."""
    built, ret = [], []
    for j in jobs:
        q, k, wq, wk = j["q"], j["k"], j["wq"], j["wk"]
        _check(q, "q", _BF16, 2)
        _check(k, "k", _BF16, 2)
        if q.shape != k.shape:
            raise ValueError("q and k must have the same shape")
        T, D = q.shape
        for t, n in ((wq, "wq"), (wk, "wk")):
            _vec(t, n, D)
        qo, ko = j.get("out") or (q, k)
        for t, n in ((qo, "q_out"), (ko, "k_out")):
            _check(t, n, _BF16, 2)
            if t.shape != q.shape:
                raise ValueError(f"{n} must have q's shape {tuple(q.shape)}")
        built.append(_lib.QkNormJob(_ptr(q), _rows(q, "q"), _ptr(k), _rows(k, "k"), _ptr(qo), _rows(qo, "q_out"),
                                    _ptr(ko), _rows(ko, "k_out"), _ptr(wq), _ptr(wk), T, D, int(j["head_dim"]),
                                    int(bool(j.get("per_head", False))), float(j.get("eps", 1e-6))))
        ret.append((qo, ko))
    _disjoint_jobs("qk_norm_multi", [(r, (j["q"], j["k"], j["wq"], j["wk"])) for j, r in zip(jobs, ret)])
    arr = (_lib.QkNormJob * len(built))(*built)
    _lib.call("ditk_qk_norm_multi", arr, len(built), _stream())
    return ret


def qk_norm_rope_(q, k, wq, wk, head_dim, eps=1e-6, per_head=False, rope=None, out=None):
    """In place: RMSNorm(q), RMSNorm(k) (across all heads, or per head) then 3D RoPE.

    q, k: [T, D] bf16 row views (e.g. column slices of a fused QKV buffer).
    out: optional (q_out, k_out) [T, D] bf16 row views written instead (q, k
    then stay untouched); returns the tensors written.
    The reference's `fused_qk_norm_rope` slot contract
    (workers/xfuser/model_executor/models/transformers/transformer_wan.py:24-25,111-115)."""
    _check(q, "q", _BF16, 2)
    _check(k, "k", _BF16, 2)
    if q.shape != k.shape:
        raise ValueError("q and k must have the same shape")
    T, D = q.shape
    ldq, ldk = _rows(q, "q"), _rows(k, "k")
    for t, n in ((wq, "wq"), (wk, "wk")):
        _vec(t, n, D)
    if rope is None:
        args = (None, None, 0, None, None, 0, 0, 0)
    else:
        if rope.segments.total != T:
            raise ValueError("rope segments do not cover q")
        if rope.cos.shape[1] != head_dim // 2:
            raise ValueError(f"RoPE tables hold {rope.cos.shape[1]} pairs, head_dim {head_dim} needs {head_dim // 2}")
        args = (_ptr(rope.cos), _ptr(rope.sin), rope.cos.shape[0], _ptr(rope.segments.dev), _ptr(rope.grids),
                rope.segments.nseg, rope.t_pairs, rope.h_pairs)
    if out is None:
        _lib.call("ditk_qk_norm_rope", _ptr(q), ldq, _ptr(k), ldk, T, D, head_dim, _ptr(wq), _ptr(wk), float(eps),
                  int(bool(per_head)), *args, _stream())
        return q, k
    qo, ko = out
    for t, n in ((qo, "q_out"), (ko, "k_out")):
        _check(t, n, _BF16, 2)
        if t.shape != q.shape:
            raise ValueError(f"{n} must have q's shape {tuple(q.shape)}")
    _lib.call("ditk_qk_norm_rope_out", _ptr(q), ldq, _ptr(k), ldk, _ptr(qo), _rows(qo, "q_out"), _ptr(ko),
              _rows(ko, "k_out"), T, D, head_dim, _ptr(wq), _ptr(wk), float(eps), int(bool(per_head)), *args,
              _stream())
    return qo, ko


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------

def _linear_args(x, w, b, epilogue, residual, gate, segments, out):
    """Checks one product's operands; returns (out, ditk_gemm's operand arguments
    without the epilogue and stream, N, K)."""
    _check(x, "x", _BF16, 2)
    _check(w, "w", _BF16, 2)
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"weight is {tuple(w.shape)}, input has K={K}")
    lda, ldw = _rows(x, "x"), _rows(w, "w")
    if b is not None:
        _vec(b, "bias", N)
    if epilogue not in EPILOGUES:
        raise ValueError(f"unknown epilogue {epilogue!r}")
    odt = torch.float32 if epilogue == "f32" else _BF16
    if out is None:
        out = torch.empty((M, N), dtype=odt, device=x.device)
    _check(out, "out", odt, 2)
    if out.shape != (M, N) or out.stride(1) != 1 or out.stride(0) % 8 or out.data_ptr() % 16:
        raise ValueError("out must be [M, N], unit column stride, leading dim % 8 == 0, 16-byte aligned")
    if N % 8 or K % 32:
        raise ValueError(f"linear needs N % 8 == 0 and K % 32 == 0 (got N={N}, K={K})")
    ldr, gate_stride, cu, nseg = 0, 0, None, 0
    if epilogue in ("gate_res", "res"):
        _check(residual, "residual", _BF16, 2)
        if residual.shape != (M, N) or residual.stride(1) != 1 or residual.stride(0) % 8 or residual.data_ptr() % 16:
            raise ValueError("residual must be [M, N] row-major with 16-byte aligned rows")
        ldr = residual.stride(0)
    if epilogue == "gate_res":
        _check(gate, "gate", torch.float32, 2)
        if segments is None or segments.total != M:
            raise ValueError("gated epilogue needs segments covering M rows")
        if gate.shape != (segments.nseg, N) or gate.stride(1) != 1 or gate.stride(0) % 4 or gate.data_ptr() % 16:
            raise ValueError(f"gate must be [{segments.nseg}, {N}] with unit column stride and 16-byte aligned rows")
        gate_stride, cu, nseg = gate.stride(0), segments.dev, segments.nseg
    return out, (_ptr(x), lda, _ptr(w), ldw, _ptr(b), _ptr(out), out.stride(0), M, _ptr(residual), ldr, _ptr(gate),
                 gate_stride, _ptr(cu), nseg), N, K


def linear(x, w, b=None, epilogue="bias", residual=None, gate=None, segments=None, out=None):
    """out = epilogue(x @ w.T + b) on MFMA.

    x [M, K] bf16 (row view), w [N, K] bf16, b [N] fp32.  Epilogues: "bias",
    "gelu" (GELU-tanh), "gate_res" (residual + bf16(y) * gate[seg]), "res"
    (residual + bf16(y)), "f32" (fp32 output), "silu"."""
    out, a, N, K = _linear_args(x, w, b, epilogue, residual, gate, segments, out)
    (xp, lda, wp, ldw, bp, op, ldc, M, rp, ldr, gp, gate_stride, cup, nseg) = a
    _lib.call("ditk_gemm", xp, lda, wp, ldw, bp, op, ldc, M, N, K, EPILOGUES[epilogue], rp, ldr, gp, gate_stride,
              cup, nseg, _stream())
    return out


def _extent(t):
    """[first, last) byte range a strided view touches (0-size views touch nothing)."""
    if t.numel() == 0:
        return 0, 0
    span = 1 + sum((n - 1) * st for n, st in zip(t.shape, t.stride()))
    return t.data_ptr(), t.data_ptr() + span * t.element_size()


def _overlap(a, b):
    a0, a1 = _extent(a)
    b0, b1 = _extent(b)
    return a0 < b1 and b0 < a1


def _disjoint_jobs(fn, jobs_io):
    """jobs_io: per job (outputs, operands).  The jobs of one launch run
    concurrently, so no job's output may overlap another job's operands or
    outputs (its own operands it may overwrite in place)."""
    for i, (outs, _) in enumerate(jobs_io):
        for j, (outs_j, ops_j) in enumerate(jobs_io):
            if i == j:
                continue
            for o in outs:
                for t in (*outs_j, *ops_j):
                    if t is not None and _overlap(o, t):
                        raise ValueError(f"{fn}: job {i}'s output overlaps a tensor of job {j}")


def linear_pair(p0, p1, epilogue="bias"):
    """Two linear() products of the same N, K and epilogue (e.g. an SD3.5 block's
    image and text projections), in one launch when their tiles fit the larger
    one's rounds.  p0, p1: dicts of linear()'s arguments (x, w, and optionally b,
    residual, gate, segments, out).  Returns (out0, out1), each bitwise what
    linear() returns for it.  Each output may alias its own residual, but neither
    output may overlap any operand or the output of the other product."""
    def args(p):
        return _linear_args(p["x"], p["w"], p.get("b"), epilogue, p.get("residual"), p.get("gate"),
                            p.get("segments"), p.get("out"))
    o0, a0, N0, K0 = args(p0)
    o1, a1, N1, K1 = args(p1)
    if (N0, K0) != (N1, K1):
        raise ValueError(f"linear_pair needs one N and K (got {N0}x{K0} and {N1}x{K1})")
    # the two products' tiles run concurrently in one launch or in order in two,
    # whichever pays: one product's output may not overlap the other's operands
    for out, other, name in ((o0, p1, "second"), (o1, p0, "first")):
        for key in ("x", "w", "b", "residual", "gate", "out"):
            t = other.get(key) if key != "out" else (o1 if out is o0 else o0)
            if t is not None and _overlap(out, t):
                raise ValueError(f"linear_pair: an output overlaps the {name} product's {key}")
    _lib.call("ditk_gemm_pair", *a0, *a1, N0, K0, EPILOGUES[epilogue], _stream())
    return o0, o1


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def vt_columns(tk, nseg):
    return int(_lib.load().ditk_vt_columns(int(tk), int(nseg)))


def transpose_v(v, heads, head_dim, segments, out=None):
    """V [Tk, heads*head_dim] -> Vt [heads, head_dim, cols] with per-segment 64-aligned columns."""
    _check(v, "v", _BF16, 2)
    ldv = _rows(v, "v")
    if v.shape[1] != heads * head_dim:
        raise ValueError(f"v must have heads * head_dim = {heads * head_dim} columns, got {v.shape[1]}")
    if segments.total != v.shape[0]:
        raise ValueError(f"segments cover {segments.total} keys, v has {v.shape[0]} rows")
    cols = vt_columns(v.shape[0], segments.nseg)
    if out is None:
        out = torch.empty((heads, head_dim, cols), dtype=_BF16, device=v.device)
    _check(out, "out", _BF16, 3)
    if out.shape != (heads, head_dim, cols) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous [{heads}, {head_dim}, {cols}] buffer")
    _lib.call("ditk_transpose_v", _ptr(v), ldv, _ptr(out), cols, v.shape[0], heads, head_dim,
              _ptr(segments.dev), segments.nseg, _stream())
    return out


LOG2E = 1.4426950408889634


def flash_attn_varlen(q, k, v, seg_q, seg_k, heads, head_dim, softmax_scale=None, return_lse=False,
                      out=None, vt=None, q_prescaled=False):
    """Block-diagonal varlen attention on packed row views.

    q [Tq, heads*head_dim], k/v [Tk, heads*head_dim] bf16 (row strides may
    differ, e.g. slices of a fused QKV buffer).  Returns out [Tq, heads*head_dim]
    (and lse [heads, Tq] fp32, natural log, when return_lse).  q_prescaled: q
    already holds q * softmax_scale * log2(e), as a QK-norm whose weight carries
    that factor produces it (the kernel then skips its per-score scaling);
    softmax_scale must be None."""
    _check(q, "q", _BF16, 2)
    _check(k, "k", _BF16, 2)
    width = heads * head_dim
    if q.shape[1] != width or k.shape[1] != width:
        raise ValueError(f"q/k must have {width} columns")
    if seg_q.nseg != seg_k.nseg:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must describe the same number of segments")
    if seg_q.total != q.shape[0] or seg_k.total != k.shape[0]:
        raise ValueError("cu_seqlens totals must match the packed token counts")
    ldq, ldk = _rows(q, "q"), _rows(k, "k")
    if vt is not None:
        _check(vt, "vt", _BF16, 3)
        if vt.shape[:2] != (heads, head_dim) or not vt.is_contiguous() or vt.shape[2] < vt_columns(k.shape[0], seg_k.nseg):
            raise ValueError("vt must be a contiguous [heads, head_dim, >= vt_columns(Tk, nseg)] buffer")
    else:
        _check(v, "v", _BF16, 2)
        if v.shape != k.shape:
            raise ValueError("v must match k")
        vt = transpose_v(v, heads, head_dim, seg_k)
    Tq = q.shape[0]
    if out is None:
        out = torch.empty((Tq, width), dtype=_BF16, device=q.device)
    _check(out, "out", _BF16, 2)
    if out.shape != (Tq, width):
        raise ValueError(f"out must be [{Tq}, {width}], got {tuple(out.shape)}")
    ldo = _rows(out, "out")
    lse = torch.empty((heads, Tq), dtype=torch.float32, device=q.device) if return_lse else None
    # with no keys at all no K tile is read: any valid address stands in for the empty K
    kp = _ptr(k) if k.shape[0] else _ptr(vt)
    if q_prescaled:
        if softmax_scale is not None:
            raise ValueError("q_prescaled carries the softmax scale in q: pass softmax_scale=None")
        _lib.call("ditk_flash_attn_varlen_q_prescaled", _ptr(q), ldq, kp, ldk, _ptr(vt), vt.shape[2],
                  _ptr(out), ldo, _ptr(lse), Tq, _ptr(seg_q.dev), _ptr(seg_k.dev), seg_q.nseg, Tq, heads,
                  head_dim, _stream())
        return (out, lse) if return_lse else out
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else float(softmax_scale)
    _lib.call("ditk_flash_attn_varlen", _ptr(q), ldq, kp, ldk, _ptr(vt), vt.shape[2], _ptr(out), ldo,
              _ptr(lse), Tq, _ptr(seg_q.dev), _ptr(seg_k.dev), seg_q.nseg, Tq, heads, head_dim, scale, _stream())
    return (out, lse) if return_lse else out


# ---------------------------------------------------------------------------
# prelude / epilogue glue
# ---------------------------------------------------------------------------

def patchify(latent, patch):
    """latent [C, F, H, W] bf16 -> [S, C*pt*ph*pw] bf16 (Conv3d-weight feature order)."""
    _check(latent, "latent", _BF16, 4)
    latent = latent.contiguous()
    C, F, H, W = latent.shape
    pt, ph, pw = patch
    out = torch.empty(((F // pt) * (H // ph) * (W // pw), C * pt * ph * pw), dtype=_BF16, device=latent.device)
    _lib.call("ditk_patchify", _ptr(latent), _ptr(out), C, F, H, W, pt, ph, pw, _stream())
    return out


def unpatchify(x, grid, patch, channels):
    """x [S, pt*ph*pw*C] bf16 -> fp32 latent [C, F'*pt, H'*ph, W'*pw]."""
    _check(x, "x", _BF16, 2)
    ldx = x.stride(0)
    Fp, Hp, Wp = grid
    pt, ph, pw = patch
    if x.shape != (Fp * Hp * Wp, pt * ph * pw * channels) or x.stride(1) != 1:
        raise ValueError(f"x must be [{Fp * Hp * Wp}, {pt * ph * pw * channels}] with unit column stride, "
                         f"got {tuple(x.shape)}")
    out = torch.empty((channels, Fp * pt, Hp * ph, Wp * pw), dtype=torch.float32, device=x.device)
    _lib.call("ditk_unpatchify", _ptr(x), ldx, _ptr(out), channels, Fp, Hp, Wp, pt, ph, pw, _stream())
    return out


def timestep_embedding(t, dim=256, max_period=10000.0):
    """Sinusoidal [N, dim] bf16, cos half first (flip_sin_to_cos=True, shift 0)."""
    _check(t, "t", torch.float32)
    t = t.reshape(-1).contiguous()
    out = torch.empty((t.numel(), dim), dtype=_BF16, device=t.device)
    _lib.call("ditk_timestep_embedding", _ptr(t), _ptr(out), t.numel(), dim, float(max_period), _stream())
    return out


def cfg_combine(cond, uncond, guidance):
    """uncond + g * (cond - uncond), fp32."""
    _check(cond, "cond", torch.float32)
    _check(uncond, "uncond", torch.float32)
    if cond.shape != uncond.shape:
        raise ValueError(f"cond and uncond shapes differ: {tuple(cond.shape)} vs {tuple(uncond.shape)}")
    out = torch.empty_like(cond, memory_format=torch.contiguous_format)
    _lib.call("ditk_cfg_combine", _ptr(cond.contiguous()), _ptr(uncond.contiguous()), _ptr(out), cond.numel(),
              float(guidance), _stream())
    return out


def solver_step(x, cond, coef, uncond=None, x_last=None, m_prev=None, m_prev2=None, x_next=None, x_corr=None,
                m_out=None):
    """Fused CFG combine + solver update (ditk_solver_step) on fp32 latents.

    coef: 11 floats {g, sigma, ax, a0, a1, a2, a3, b0, b1, b2, bv}.  Returns x_next
    (new tensor unless given; may be x itself)."""
    if len(coef) != 11:
        raise ValueError("solver_step: coef needs 11 values")
    _check(x, "x", torch.float32)
    _check(cond, "cond", torch.float32)
    n = x.numel()
    for name, t in (("cond", cond), ("uncond", uncond), ("x_last", x_last), ("m_prev", m_prev),
                    ("m_prev2", m_prev2), ("x_next", x_next), ("x_corr", x_corr), ("m_out", m_out)):
        if t is not None:
            _check(t, name, torch.float32)
            if t.numel() != n or not t.is_contiguous():
                raise ValueError(f"solver_step: {name} must be contiguous with {n} elements")
    if not x.is_contiguous():
        raise ValueError("solver_step: x must be contiguous")
    if x_next is None:
        x_next = torch.empty_like(x)
    arr = (ctypes.c_float * 11)(*[float(c) for c in coef])
    opt = lambda t: _ptr(t) if t is not None else None  # noqa: E731
    _lib.call("ditk_solver_step", _ptr(x), _ptr(cond), opt(uncond), opt(x_last), opt(m_prev), opt(m_prev2),
              _ptr(x_next), opt(x_corr), opt(m_out), n, ctypes.addressof(arr), _stream())
    return x_next


def joint_gather(img, txt, seg_img, seg_txt, out=None):
    """Interleave per segment: [img rows of m, txt rows of m] -> joint [Ti+Tt, W]."""
    total, width = _joint_copy_check(img, txt, seg_img, seg_txt)
    if out is None:
        out = torch.empty((total, width), dtype=_BF16, device=img.device)
    _joint_rows_check(out, "out", total, width)
    _lib.call("ditk_joint_copy", _ptr(img), img.stride(0), _ptr(txt), txt.stride(0), _ptr(out), out.stride(0),
              _ptr(seg_img.dev), _ptr(seg_txt.dev), seg_img.nseg, total, width, 0, _stream())
    return out


def _joint_rows_check(t, name, rows, width):
    _check(t, name, _BF16, 2)
    _rows(t, name)
    if t.shape != (rows, width):
        raise ValueError(f"{name} must be [{rows}, {width}], got {tuple(t.shape)}")


def _joint_copy_check(img, txt, seg_img, seg_txt):
    """Operands of a joint gather / scatter: image rows [seg_img.total, W] and text
    rows [seg_txt.total, W], both bf16 row views; returns (joint rows, W)."""
    if seg_img.nseg != seg_txt.nseg:
        raise ValueError("image and text segment tables must have the same number of segments")
    _check(img, "img", _BF16, 2)
    width = img.shape[1]
    _joint_rows_check(img, "img", seg_img.total, width)
    _joint_rows_check(txt, "txt", seg_txt.total, width)
    return seg_img.total + seg_txt.total, width


def _joint_tables(seg_img, seg_txt, seg_joint):
    if not (seg_img.nseg == seg_txt.nseg == seg_joint.nseg):
        raise ValueError("image, text and joint segment tables must have the same number of segments")
    if list(seg_joint.cu) != [int(a) + int(b) for a, b in zip(seg_img.cu, seg_txt.cu)]:
        raise ValueError("joint segments must be cu_joint = cu_img + cu_txt")


def transpose_v_joint(v_img, v_txt, heads, head_dim, seg_img, seg_txt, seg_joint):
    """transpose_v of the joint rows (image rows of m, then text rows of m) read
    straight from the two sources; the layout ditk_transpose_v gives the gathered V."""
    _check(v_img, "v_img", _BF16, 2)
    _check(v_txt, "v_txt", _BF16, 2)
    _joint_tables(seg_img, seg_txt, seg_joint)
    if v_img.shape != (seg_img.total, heads * head_dim) or v_txt.shape != (seg_txt.total, heads * head_dim):
        raise ValueError("v_img / v_txt must be [segment total, heads*head_dim]")
    ldv = _rows(v_img, "v_img")
    if _rows(v_txt, "v_txt") != ldv:
        raise ValueError("v_img and v_txt must share a row stride")
    T = seg_joint.total
    cols = vt_columns(T, seg_joint.nseg)
    vt = torch.empty((heads, head_dim, cols), dtype=_BF16, device=v_img.device)
    _lib.call("ditk_transpose_v_joint", _ptr(v_img), _ptr(v_txt), ldv, _ptr(vt), cols, T, heads, head_dim,
              _ptr(seg_img.dev), _ptr(seg_txt.dev), _ptr(seg_joint.dev), seg_joint.nseg, _stream())
    return vt


def joint_attention_q_prescaled(q_img, q_txt, k_img, k_txt, vt, seg_img, seg_txt, seg_joint, heads, head_dim,
                                out_img=None, out_txt=None):
    """Joint attention straight from the image and text projections (head_dim 64,
    q pre-scaled by softmax_scale * log2(e), vt from transpose_v_joint): joint
    segment m = image rows of m, then text rows of m.  Returns (o_img, o_txt),
    bitwise equal to joint_gather -> flash_attn_varlen(q_prescaled=True) ->
    joint_scatter."""
    width = heads * head_dim
    if head_dim != 64:
        raise ValueError("joint attention from two sources needs head_dim 64")
    _joint_tables(seg_img, seg_txt, seg_joint)
    for a, b, t in ((q_img, q_txt, "q"), (k_img, k_txt, "k")):
        _check(a, t + "_img", _BF16, 2)
        _check(b, t + "_txt", _BF16, 2)
        if a.shape != (seg_img.total, width) or b.shape != (seg_txt.total, width):
            raise ValueError(f"{t}_img / {t}_txt must be [segment total, {width}]")
        if _rows(a, t + "_img") != _rows(b, t + "_txt"):
            raise ValueError(f"{t}_img and {t}_txt must share a row stride")
    T = seg_joint.total
    _check(vt, "vt", _BF16, 3)
    if vt.shape[:2] != (heads, head_dim) or not vt.is_contiguous() or vt.shape[2] < vt_columns(T, seg_joint.nseg):
        raise ValueError("vt must be a contiguous [heads, head_dim, >= vt_columns(T_joint, nseg)] buffer")
    if out_img is None:
        out_img = torch.empty((seg_img.total, width), dtype=_BF16, device=q_img.device)
    if out_txt is None:
        out_txt = torch.empty((seg_txt.total, width), dtype=_BF16, device=q_img.device)
    for t, n, rows in ((out_img, "out_img", seg_img.total), (out_txt, "out_txt", seg_txt.total)):
        _check(t, n, _BF16, 2)
        if t.shape != (rows, width):
            raise ValueError(f"{n} must be [{rows}, {width}], got {tuple(t.shape)}")
    if _rows(out_img, "out_img") != _rows(out_txt, "out_txt"):
        raise ValueError("out_img and out_txt must share a row stride")
    _lib.call("ditk_joint_attn_q_prescaled", _ptr(q_img), _ptr(q_txt), _rows(q_img, "q_img"), _ptr(k_img),
              _ptr(k_txt), _rows(k_img, "k_img"), _ptr(vt), vt.shape[2], _ptr(out_img), _ptr(out_txt),
              _rows(out_img, "out_img"), _ptr(seg_img.dev), _ptr(seg_txt.dev), _ptr(seg_joint.dev),
              seg_joint.nseg, T, heads, head_dim, _stream())
    return out_img, out_txt


def joint_scatter(joint, img, txt, seg_img, seg_txt):
    """Inverse of joint_gather: joint rows back into img / txt buffers."""
    total, width = _joint_copy_check(img, txt, seg_img, seg_txt)
    _joint_rows_check(joint, "joint", total, width)
    _lib.call("ditk_joint_copy", _ptr(img), img.stride(0), _ptr(txt), txt.stride(0), _ptr(joint),
              joint.stride(0), _ptr(seg_img.dev), _ptr(seg_txt.dev), seg_img.nseg, total, joint.shape[1], 1,
              _stream())
    return img, txt


def silu(x):
    _check(x, "x", _BF16)
    x = x.contiguous()
    out = torch.empty_like(x)
    _lib.call("ditk_silu", _ptr(x), _ptr(out), x.numel(), _stream())
    return out
