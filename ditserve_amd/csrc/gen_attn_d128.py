"""Generate the instruction body of the head_dim-128 varlen flash-attention
kernel (attention.hip: flash_fwd_d128) as gfx950 assembly.

Why generated assembly: the kernel runs one wave per SIMD with 64 queries per
wave, which needs about 460 registers per lane.  The compiler cannot place that
working set (its allocation spills or shuffles AGPR<->VGPR copies), so the
registers are assigned here by hand:

  VGPR v0..v63     S set A   S^T accumulators [qb][kk] (16 each) of one key tile
  VGPR v64..v127   S set B   (the loop is unrolled by two so that the tile being
                             computed and the tile being exponentiated alternate)
  VGPR v128..v159  P set A   bf16 P^T fragments [qb][g] (4 dwords each)
  VGPR v160..v191  P set B
  VGPR v192..v199  exp temporaries (a ring of four score pairs)
  VGPR v200..v201  rs0[qb]   row sums of keys 0..31 of the pending tile
  VGPR v202..v203  rs1[qb]   row sums of keys 32..63
  VGPR v204..v205  negm[qb]  minus the running max (log2 units)
  VGPR v206..v207  l[qb]     running softmax denominators
  VGPR v208..v211  K fragment LDS read addresses (per chunk residue c % 4)
  VGPR v212..v215  Vt fragment LDS read addresses (per key group g)
  VGPR v216..v219  DMA address temporaries
  AGPR a0..a127    O^T accumulators [qb][d] (16 each)
  AGPR a128..a191  Q fragments [qb][c] (4 each)
  AGPR a192..a215  K fragment ring: 3 chunks x 2 (kk)
  AGPR a216..a231  Vt fragment ring: 4 fragments

Per 64-key tile kt the wave (queries q0..q0+63 of one (segment, head)) runs
  phase 1: S(kt+1) = K(kt+1) Q^T    (32 MFMAs)  ||  P(kt) keys 32..63 (VALU)
  check:   lazy-rescale test on the row sums of P(kt)
  phase 2: O += Vt(kt) P(kt)        (32 MFMAs)  ||  P(kt+1) keys 0..31 (VALU)
with one VALU half-item per MFMA slot, K fragments read two chunks ahead and
Vt fragments three fragments ahead, and the next tiles' K and Vt streamed into
LDS by direct global->LDS DMA.  The arithmetic per score, the order of every
row sum and the rescale rule are those of the C++ kernel
(flash_fwd_kernel<128, 8, 1>), so the two agree bitwise.

Hazards the hardware does not interlock are covered explicitly: an s_nop before
VALU reads of MFMA results and before MFMAs read AGPRs written by
v_accvgpr_write, an s_nop between an M0 write and the DMA that reads it.

Usage: python gen_attn_d128.py [out.inc]  (writes attn_d128_body.inc beside it)
"""
import os
import sys

# ----------------------------------------------------------------------------
# register map
S_SET = (0, 64)
P_SET = (128, 160)
TMP = 192
RS0, RS1, NEGM, LRUN = 200, 202, 204, 206
KADDR, VADDR, DTMP = 208, 212, 216
O_A, Q_A, KF_A, VF_A = 0, 128, 192, 216
LAST_VGPR, LAST_AGPR = 219, 231

# scalar registers owned by the body (all callee state lives in these)
S_KDMA = 60      # s[60:61] K DMA base (bytes) of tile kt+2
S_VDMA = 62      # s[62:63] Vt DMA base (bytes) of tile kt+1
S_KST = 64       # s64 LDS base of the K stage read this tile, s65 the DMA stage
S_VST = 66       # s66 Vt stage read this tile, s67 Vt DMA stage
S_KT = 68        # s68 tile index kt
S_ROWLIM = 69    # s69 last valid row of the K tile being DMA'd
S_T0, S_T1, S_T2, S_T3 = 70, 71, 72, 73
S_CMP = 74       # s[74:75] compare mask
S_EXEC = 76      # s[76:77] saved exec
S_VALID = 78     # s78 valid keys of the last tile
S_M0 = 79        # s79 M0 staging
S_V3 = 80        # s80 the third Vt stage (read two tiles from now)
SGPRS = list(range(60, 81))

BN, HD = 64, 128
# schedule options (the defaults are the shipped schedule)
OPTS = {"p2wait": 2, "dma_slots": True, "barrier_slot": 32}
KSTAGE_BYTES = BN * HD * 2     # 16 KiB
VSTAGE_BYTES = HD * BN * 2     # 16 KiB


def s_(n):
    return f"s{n}"


def sp(n):
    return f"s[{n}:{n + 1}]"


def vr(lo, n=1):
    return f"v{lo}" if n == 1 else f"v[{lo}:{lo + n - 1}]"


def ar(lo, n=1):
    return f"a{lo}" if n == 1 else f"a[{lo}:{lo + n - 1}]"


def s_reg(setv, qb, kk, v=None):
    base = S_SET[setv] + qb * 32 + kk * 16
    return base if v is None else base + v


def p_reg(setv, qb, g, e=0):
    return P_SET[setv] + qb * 16 + g * 4 + e


def o_reg(qb, d):
    return O_A + (qb * 4 + d) * 16


def q_reg(qb, c):
    return Q_A + (qb * 8 + c) * 4


def kf_reg(r, kk):
    return KF_A + (r * 2 + kk) * 4


def vf_reg(r):
    return VF_A + r * 4


class Gen:
    def __init__(self):
        self.lines = []
        self.label_n = 0
        self.lds = []

    def __call__(self, s):
        self.lines.append(s)

    def label(self, name):
        self.lines.append(f"{name}:")

    def new_label(self, stem):
        self.label_n += 1
        return f"L_{stem}_{self.label_n}_%="

    # Outstanding LDS reads, oldest first.  LDS returns in order, so waiting for
    # one read means allowing only the reads issued after it to be pending.
    def lds_issue(self, tag):
        self.lds.append(tag)

    def lds_wait(self, tag):
        if tag not in self.lds:
            return
        i = self.lds.index(tag)
        self(f"s_waitcnt lgkmcnt({min(len(self.lds) - i - 1, 15)})")
        del self.lds[:i + 1]

    def lds_wait_all(self):
        self("s_waitcnt lgkmcnt(0)")
        self.lds = []

    def nops(self, n):
        while n > 0:
            k = min(n, 8)
            self(f"s_nop {k - 1}")
            n -= k


# ----------------------------------------------------------------------------
# pieces

def pair_list(kk):
    """The 16 score pairs of one key half (kk) of a tile for both query blocks,
    in the C++ kernel's order: qb-major, then j, then e."""
    return [(qb, kk, j, e) for qb in range(2) for j in range(2) for e in range(4)]


def item_order(n):
    """Half-item sequence over n pairs: a0 a1 b0 a2 b1 ... a(n-1) b(n-2) b(n-1)."""
    out = []
    for k in range(2 * n):
        if k == 0:
            out.append((0, 0))
        elif k == 2 * n - 1:
            out.append((1, n - 1))
        elif k & 1:
            out.append((0, (k + 1) // 2))
        else:
            out.append((1, k // 2 - 1))
    return out


def emit_half(g, half, pi, pair, s_set, p_set, rs_base):
    """One half-item: 'a' = two fma + two exp2 into the temp ring, 'b' = pack into
    P, and the row sum rs += (p0 + p1)."""
    qb, kk, j, e = pair
    t0 = TMP + 2 * (pi % 4)
    t1 = t0 + 1
    if half == 0:
        s0 = s_reg(s_set, qb, kk, j * 8 + 2 * e)
        g(f"v_fma_f32 {vr(t0)}, {vr(s0)}, %[sc], {vr(NEGM + qb)}")
        g(f"v_fma_f32 {vr(t1)}, {vr(s0 + 1)}, %[sc], {vr(NEGM + qb)}")
        g(f"v_exp_f32 {vr(t0)}, {vr(t0)}")
        g(f"v_exp_f32 {vr(t1)}, {vr(t1)}")
    else:
        g(f"v_cvt_pk_bf16_f32 {vr(p_reg(p_set, qb, kk * 2 + j, e))}, {vr(t0)}, {vr(t1)}")
        g(f"v_add_f32 {vr(t0)}, {vr(t0)}, {vr(t1)}")
        g(f"v_add_f32 {vr(rs_base + qb)}, {vr(rs_base + qb)}, {vr(t0)}")


def set_m0(g, sreg_expr):
    g(f"s_mov_b32 m0, {sreg_expr}")
    g("s_nop 0")


def kdma(g, i):
    """DMA instruction i (0..3) of this wave for the K tile at S_KDMA into the K
    DMA stage: rows min(krow_i, rowlim), 16 bytes per lane."""
    t = DTMP + i
    g(f"v_min_u32 {vr(t)}, %[krow{i}], {s_(S_ROWLIM)}")
    g(f"v_mad_u32_u24 {vr(t)}, {vr(t)}, %[ldkb], %[kcolb{i}]")
    g(f"s_add_u32 {s_(S_M0)}, {s_(S_KST + 1)}, {i * 4096}")
    g(f"s_add_u32 {s_(S_M0)}, {s_(S_M0)}, %[wave1k]")
    set_m0(g, s_(S_M0))
    g(f"global_load_lds_dwordx4 {vr(t)}, {sp(S_KDMA)}")


def kdma_addr(g, i):
    t = DTMP + i
    g(f"v_min_u32 {vr(t)}, %[krow{i}], {s_(S_ROWLIM)}")
    g(f"v_mad_u32_u24 {vr(t)}, {vr(t)}, %[ldkb], %[kcolb{i}]")


def kdma_issue(g, i):
    g(f"s_add_u32 {s_(S_M0)}, {s_(S_KST + 1)}, {i * 4096}")
    g(f"s_add_u32 {s_(S_M0)}, {s_(S_M0)}, %[wave1k]")
    set_m0(g, s_(S_M0))
    g(f"global_load_lds_dwordx4 {vr(DTMP + i)}, {sp(S_KDMA)}")


def vdma(g, i):
    g(f"s_add_u32 {s_(S_M0)}, {s_(S_VST + 1)}, {i * 4096}")
    g(f"s_add_u32 {s_(S_M0)}, {s_(S_M0)}, %[wave1k]")
    set_m0(g, s_(S_M0))
    g(f"global_load_lds_dwordx4 %[voff{i}], {sp(S_VDMA)}")


def k_read(g, chunk, kk, stage_in_addr=True):
    """ds_read of K fragment (chunk, kk) from the K stage whose base is folded into
    the KADDR registers."""
    off = (chunk >> 2) * 8192 + kk * 4096
    g(f"ds_read_b128 {ar(kf_reg(chunk % 3, kk), 4)}, {vr(KADDR + (chunk & 3))} offset:{off}")
    g.lds_issue(("k", chunk, kk))


def v_read(g, f):
    grp, d = f // 4, f % 4
    g(f"ds_read_b128 {ar(vf_reg(f % 4), 4)}, {vr(VADDR + grp)} offset:{d * 4096}")
    g.lds_issue(("v", f))


def mfma_s(g, s_set, qb, kk, chunk):
    dst = s_reg(s_set, qb, kk)
    src_c = "0" if chunk == 0 else vr(dst, 16)
    g(f"v_mfma_f32_32x32x16_bf16 {vr(dst, 16)}, {ar(kf_reg(chunk % 3, kk), 4)}, {ar(q_reg(qb, chunk), 4)}, {src_c}")


def mfma_o(g, p_set, qb, d, grp, ring):
    o = o_reg(qb, d)
    g(f"v_mfma_f32_32x32x16_bf16 {ar(o, 16)}, {ar(vf_reg(ring), 4)}, {vr(p_reg(p_set, qb, grp), 4)}, {ar(o, 16)}")


def set_addrs(g, k_stage_sreg, v_stage_sreg):
    for i in range(4):
        g(f"v_add_u32 {vr(KADDR + i)}, {s_(k_stage_sreg)}, %[kbase{i}]")
    for i in range(4):
        g(f"v_add_u32 {vr(VADDR + i)}, {s_(v_stage_sreg)}, %[vbase{i}]")


def s_phase(g, s_set, items=None, dma=None, vreads_after=True):
    """32 S MFMAs (S(kt+1) into s_set) with K fragments two chunks ahead; the
    first two chunks' reads must already be issued.  items: list of callables,
    one per slot; dma: list of callables for the first slots."""
    slot = 0
    for c in range(8):
        g.lds_wait(("k", c, 1))
        for kk in range(2):
            for qb in range(2):
                mfma_s(g, s_set, qb, kk, c)
                if kk == 0 and qb == 0 and c + 2 < 8:
                    k_read(g, c + 2, 0)
                    k_read(g, c + 2, 1)
                if kk == 0 and qb == 0 and c == 7 and vreads_after:
                    for f in range(3):
                        v_read(g, f)
                if dma is not None and slot < len(dma):
                    dma[slot]()
                if items is not None:
                    items[slot]()
                slot += 1


def o_phase(g, p_set, items=None, hooks=None):
    """32 PV MFMAs with Vt fragments three ahead (the first three already issued);
    hooks: {slot: callable} run before that slot's MFMA."""
    slot = 0
    for f in range(16):
        grp, d = f // 4, f % 4
        for qb in range(2):
            if hooks and slot in hooks:
                hooks[slot]()
            if qb == 0:
                g.lds_wait(("v", f))
            mfma_o(g, p_set, qb, d, grp, f % 4)
            if qb == 0 and f + 3 < 16:
                v_read(g, f + 3)
            if items is not None:
                items[slot]()
            slot += 1


def make_items(g, pairs, s_set, p_set, rs_base, slots=32):
    order = item_order(len(pairs))
    per = [[] for _ in range(slots)]
    for k, (half, pi) in enumerate(order):
        per[k * slots // len(order)].append((half, pi))

    def fn(lst):
        return lambda: [emit_half(g, h, pi, pairs[pi], s_set, p_set, rs_base) for h, pi in lst]
    return [fn(x) for x in per]


def row_max_to(g, s_set, qb, dst, tmp):
    """dst = max over this lane's 32 scores of query block qb (both half-waves
    combined), times the softmax scale (log2 units)."""
    base = s_reg(s_set, qb, 0)
    g(f"v_max3_f32 {vr(dst)}, {vr(base)}, {vr(base + 16)}, {vr(base + 1)}")
    for v in range(1, 16):
        a, b = base + v, base + 16 + v
        if v == 1:
            g(f"v_max_f32 {vr(dst)}, {vr(dst)}, {vr(b)}")
        else:
            g(f"v_max3_f32 {vr(dst)}, {vr(dst)}, {vr(a)}, {vr(b)}")
    g(f"ds_bpermute_b32 {vr(tmp)}, %[xaddr], {vr(dst)}")
    g("s_waitcnt lgkmcnt(0)")
    g(f"v_max_f32 {vr(dst)}, {vr(dst)}, {vr(tmp)}")
    g(f"v_mul_f32 {vr(dst)}, %[sc], {vr(dst)}")


def scale_o(g, qb, alpha):
    for d in range(4):
        for v in range(16):
            a = o_reg(qb, d) + v
            g(f"v_accvgpr_read_b32 {vr(DTMP)}, {ar(a)}")
            g(f"v_mul_f32 {vr(DTMP)}, {vr(DTMP)}, {vr(alpha)}")
            g(f"v_accvgpr_write_b32 {ar(a)}, {vr(DTMP)}")


def softmax_tile(g, s_set, p_set, qb, kks, rs_dst, masked=False):
    """Recompute P for the given key halves of query block qb from the raw scores
    and the running m; rs_dst += sum (masked: keys >= valid excluded)."""
    for kk in kks:
        for j in range(2):
            for e in range(4):
                s0 = s_reg(s_set, qb, kk, j * 8 + 2 * e)
                t0, t1 = TMP, TMP + 1
                g(f"v_fma_f32 {vr(t0)}, {vr(s0)}, %[sc], {vr(NEGM + qb)}")
                g(f"v_fma_f32 {vr(t1)}, {vr(s0 + 1)}, %[sc], {vr(NEGM + qb)}")
                g(f"v_exp_f32 {vr(t0)}, {vr(t0)}")
                g(f"v_exp_f32 {vr(t1)}, {vr(t1)}")
                g("s_nop 0")
                g(f"v_cvt_pk_bf16_f32 {vr(p_reg(p_set, qb, kk * 2 + j, e))}, {vr(t0)}, {vr(t1)}")
                if masked:
                    key = kk * 32 + j * 16 + 2 * e
                    # keep p where key (+1) < valid, i.e. hh8 < valid - key (- 1)
                    for t, kk_off in ((t0, 0), (t1, 1)):
                        g(f"s_sub_i32 {s_(S_T0)}, {s_(S_VALID)}, {key + kk_off}")
                        g(f"v_cmp_gt_i32 vcc, {s_(S_T0)}, %[hh8]")
                        g(f"v_cndmask_b32 {vr(t)}, 0, {vr(t)}, vcc")
                g(f"v_add_f32 {vr(t0)}, {vr(t0)}, {vr(t1)}")
                g(f"v_add_f32 {vr(rs_dst + qb)}, {vr(rs_dst + qb)}, {vr(t0)}")


def exact_rescale(g, s_set, p_set, kks, masked=False):
    """The C++ rescale: m_new = max(m, row max of the tile's scores), O and l
    scaled by exp2(m - m_new), P of the tile recomputed against m_new into rs0.
    (rs1 is cleared.)"""
    g.nops(20)  # O accumulators read below: MFMA results must have landed
    for qb in range(2):
        mx, tmp, alpha = DTMP + 1, DTMP + 2, DTMP + 3
        row_max_to(g, s_set, qb, mx, tmp)
        # m_old = -negm ; m_new = max(m_old, mx) ; alpha = exp2(m_old - m_new)
        g(f"v_sub_f32 {vr(tmp)}, 0, {vr(NEGM + qb)}")        # m_old
        g(f"v_max_f32 {vr(mx)}, {vr(tmp)}, {vr(mx)}")         # m_new
        g(f"v_sub_f32 {vr(alpha)}, {vr(tmp)}, {vr(mx)}")
        g(f"v_exp_f32 {vr(alpha)}, {vr(alpha)}")
        g(f"v_sub_f32 {vr(NEGM + qb)}, 0, {vr(mx)}")
        g("s_nop 0")
        g(f"v_mul_f32 {vr(LRUN + qb)}, {vr(LRUN + qb)}, {vr(alpha)}")
        scale_o(g, qb, alpha)
        g(f"v_mov_b32 {vr(RS0 + qb)}, 0")
        g(f"v_mov_b32 {vr(RS1 + qb)}, 0")
        softmax_tile(g, s_set, p_set, qb, kks, RS0, masked)
    g.nops(3)  # v_accvgpr_write -> MFMA srcC


def tile(g, a):
    """One steady tile kt: scores of tile kt in S set a, S(kt+1) computed into set
    1 - a.  Entered with the reads of K(kt+1) chunks 0 and 1 already issued.

    The workgroup barrier that publishes this tile's DMA (K(kt+2), Vt(kt+1)) sits
    inside phase 2, at OPTS["barrier_slot"]: the rest of phase 2 issues the next
    tile's first K reads behind the PV MFMAs, so no LDS latency is exposed at the
    tile boundary.  Vt therefore rotates through three stages: a wave past the
    barrier may DMA Vt(kt+2) while another still reads Vt(kt)."""
    b = 1 - a
    after_check = g.new_label("checked")
    resc = g.new_label("rescale")
    g.lds = [("k", 0, 0), ("k", 0, 1), ("k", 1, 0), ("k", 1, 1)]
    for i in range(4):
        g(f"v_add_u32 {vr(VADDR + i)}, {s_(S_VST)}, %[vbase{i}]")
    # DMA of K(min(kt+2, nkt-1)) (past the last tile it refetches the last one
    # into the stage of K(kt), which no wave reads any more) and of Vt(kt+1)
    g(f"s_add_u32 {s_(S_T0)}, {s_(S_KT)}, 2")
    g(f"s_sub_u32 {s_(S_T1)}, %[nkt], 1")
    g(f"s_min_u32 {s_(S_T0)}, {s_(S_T0)}, {s_(S_T1)}")
    g(f"s_cmp_eq_u32 {s_(S_T0)}, {s_(S_T1)}")
    g(f"s_cselect_b32 {s_(S_ROWLIM)}, {s_(S_VALID)}, {BN}")
    g(f"s_sub_u32 {s_(S_ROWLIM)}, {s_(S_ROWLIM)}, 1")
    g(f"s_mul_i32 {s_(S_KDMA)}, {s_(S_T0)}, %[ktile]")
    g(f"s_mul_hi_u32 {s_(S_KDMA + 1)}, {s_(S_T0)}, %[ktile]")
    g(f"s_add_u32 {s_(S_KDMA)}, {s_(S_KDMA)}, %[kdma_lo]")
    g(f"s_addc_u32 {s_(S_KDMA + 1)}, {s_(S_KDMA + 1)}, %[kdma_hi]")
    for i in range(4):
        kdma_addr(g, i)
    dmas = [(lambda i=i: kdma_issue(g, i)) for i in range(4)] + [(lambda i=i: vdma(g, i)) for i in range(4)]
    if not OPTS["dma_slots"]:
        for d in dmas:
            d()
        dmas = None
    # phase 1: S(kt+1) into set b || P(kt) keys 32..63 from set a
    g(f"v_mov_b32 {vr(RS1)}, 0")
    g(f"v_mov_b32 {vr(RS1 + 1)}, 0")
    items = make_items(g, pair_list(1), a, a, RS1)
    s_phase(g, b, items=items, dma=dmas)
    # lazy-rescale check on tile kt: rsum = rs0 + rs1 (per lane), flag !(rsum <= 256)
    for qb in range(2):
        g(f"v_add_f32 {vr(DTMP + qb)}, {vr(RS0 + qb)}, {vr(RS1 + qb)}")
    g(f"s_mov_b32 {s_(S_T2)}, 0x43800000")
    g(f"v_cmp_nge_f32 vcc, {s_(S_T2)}, {vr(DTMP)}")
    g(f"v_cmp_nge_f32_e64 {sp(S_CMP)}, {s_(S_T2)}, {vr(DTMP + 1)}")
    g(f"s_or_b64 vcc, vcc, {sp(S_CMP)}")
    g(f"s_cbranch_vccnz {resc}")
    g.label(after_check)
    for qb in range(2):
        g(f"v_add_f32 {vr(DTMP + qb)}, {vr(RS0 + qb)}, {vr(RS1 + qb)}")
        g(f"v_add_f32 {vr(LRUN + qb)}, {vr(LRUN + qb)}, {vr(DTMP + qb)}")
        g(f"v_mov_b32 {vr(RS0 + qb)}, 0")
    # phase 2: O += Vt(kt) P(kt) || P(kt+1) keys 0..31 from set b.  The wait
    # covers the VALU reads of the S(kt+1) results of the last MFMAs (already
    # three MFMAs old) and the MFMA reads of the P(kt) just packed.
    g.nops(OPTS["p2wait"])
    items = make_items(g, pair_list(0), b, b, RS0)

    def barrier():
        # publish this tile's DMA: own loads landed, then the workgroup barrier
        g("s_waitcnt vmcnt(0)")
        g("s_barrier")
        # rotate: K stages swap, Vt stages rotate, DMA base advances, kt += 1
        g(f"s_mov_b32 {s_(S_T0)}, {s_(S_KST)}")
        g(f"s_mov_b32 {s_(S_KST)}, {s_(S_KST + 1)}")
        g(f"s_mov_b32 {s_(S_KST + 1)}, {s_(S_T0)}")
        g(f"s_mov_b32 {s_(S_T0)}, {s_(S_VST)}")
        g(f"s_mov_b32 {s_(S_VST)}, {s_(S_VST + 1)}")
        g(f"s_mov_b32 {s_(S_VST + 1)}, {s_(S_V3)}")
        g(f"s_mov_b32 {s_(S_V3)}, {s_(S_T0)}")
        g(f"s_add_u32 {s_(S_VDMA)}, {s_(S_VDMA)}, {BN * 2}")
        g(f"s_addc_u32 {s_(S_VDMA + 1)}, {s_(S_VDMA + 1)}, 0")
        g(f"s_add_u32 {s_(S_KT)}, {s_(S_KT)}, 1")
        for i in range(4):
            g(f"v_add_u32 {vr(KADDR + i)}, {s_(S_KST)}, %[kbase{i}]")

    def next_reads(chunk):
        return lambda: (k_read(g, chunk, 0), k_read(g, chunk, 1))
    bs = OPTS["barrier_slot"]
    if bs < 30:
        o_phase(g, a, items=items, hooks={bs: barrier, bs + 1: next_reads(0), bs + 2: next_reads(1)})
    else:
        o_phase(g, a, items=items)
        barrier()
        next_reads(0)()
        next_reads(1)()
    return resc, after_check


def rescale_block(g, a, resc, back):
    """Out-of-line rescale of tile kt (scores still in set a, P(kt) in P set a)."""
    g.label(resc)
    exact_rescale(g, a, a, (0, 1))
    g(f"s_branch {back}")


def last_tile(g, a):
    """The last key tile (scores in set a): P of all 64 keys against m with keys
    past the segment end out of the row sums, the rescale test, then O += Vt P."""
    full = g.new_label("fullrs")
    done_rs = g.new_label("rsdone")
    resc = g.new_label("lastresc")
    checked = g.new_label("lastchecked")
    g.nops(20)
    g.lds_wait_all()
    set_addrs(g, S_KST, S_VST)
    for qb in range(2):
        g(f"v_mov_b32 {vr(RS0 + qb)}, 0")
    g(f"s_cmp_eq_u32 {s_(S_VALID)}, {BN}")
    g(f"s_cbranch_scc1 {full}")
    for qb in range(2):
        softmax_tile(g, a, a, qb, (0, 1), RS0, masked=True)
    g(f"s_branch {done_rs}")
    g.label(full)
    for qb in range(2):
        softmax_tile(g, a, a, qb, (0, 1), RS0, masked=False)
    g.label(done_rs)
    g(f"s_mov_b32 {s_(S_T2)}, 0x43800000")
    g(f"v_cmp_nge_f32 vcc, {s_(S_T2)}, {vr(RS0)}")
    g(f"v_cmp_nge_f32_e64 {sp(S_CMP)}, {s_(S_T2)}, {vr(RS0 + 1)}")
    g(f"s_or_b64 vcc, vcc, {sp(S_CMP)}")
    g(f"s_cbranch_vccz {checked}")
    # rescale against the exact tile max (masked sums)
    g(f"s_cmp_eq_u32 {s_(S_VALID)}, {BN}")
    g(f"s_cbranch_scc1 {resc}")
    exact_rescale(g, a, a, (0, 1), masked=True)
    g(f"s_branch {checked}")
    g.label(resc)
    exact_rescale(g, a, a, (0, 1), masked=False)
    g.label(checked)
    for qb in range(2):
        g(f"v_add_f32 {vr(LRUN + qb)}, {vr(LRUN + qb)}, {vr(RS0 + qb)}")
    g("s_nop 2")
    for f in range(3):
        v_read(g, f)
    o_phase(g, a, items=None)


def prologue(g):
    # scalar state
    g(f"s_mov_b32 {s_(S_KDMA)}, %[kdma_lo]")
    g(f"s_mov_b32 {s_(S_KDMA + 1)}, %[kdma_hi]")
    g(f"s_mov_b32 {s_(S_VDMA)}, %[vdma_lo]")
    g(f"s_mov_b32 {s_(S_VDMA + 1)}, %[vdma_hi]")
    g(f"s_mov_b32 {s_(S_KST)}, %[lds_k]")
    g(f"s_add_u32 {s_(S_KST + 1)}, %[lds_k], {KSTAGE_BYTES}")
    g(f"s_mov_b32 {s_(S_VST)}, %[lds_v]")
    g(f"s_add_u32 {s_(S_VST + 1)}, %[lds_v], {VSTAGE_BYTES}")
    g(f"s_add_u32 {s_(S_V3)}, %[lds_v], {2 * VSTAGE_BYTES}")
    g(f"s_mov_b32 {s_(S_KT)}, 0")
    g(f"s_mov_b32 {s_(S_VALID)}, %[valid_last]")
    # Q fragments straight into AGPRs
    for qb in range(2):
        for c in range(8):
            g(f"global_load_dwordx4 {ar(q_reg(qb, c), 4)}, %[qoff{qb}], %[qbase] offset:{c * 32}")
    # O = 0, l = 0
    for i in range(128):
        g(f"v_accvgpr_write_b32 {ar(O_A + i)}, 0")
    for qb in range(2):
        g(f"v_mov_b32 {vr(LRUN + qb)}, 0")
        g(f"v_mov_b32 {vr(RS0 + qb)}, 0")
        g(f"v_mov_b32 {vr(RS1 + qb)}, 0")
    # K(0) into stage 0 (DMA stage register temporarily = stage 0)
    g(f"s_cmp_eq_u32 %[nkt], 1")
    g(f"s_cselect_b32 {s_(S_ROWLIM)}, {s_(S_VALID)}, {BN}")
    g(f"s_sub_u32 {s_(S_ROWLIM)}, {s_(S_ROWLIM)}, 1")
    g(f"s_mov_b32 {s_(S_T3)}, {s_(S_KST + 1)}")
    g(f"s_mov_b32 {s_(S_KST + 1)}, {s_(S_KST)}")
    for i in range(4):
        kdma(g, i)
    g(f"s_mov_b32 {s_(S_KST + 1)}, {s_(S_T3)}")
    g("s_waitcnt vmcnt(0)")
    g("s_barrier")
    # K(1) into stage 1 when nkt > 1; Vt(0) into Vt stage 0
    no_k1 = g.new_label("nok1")
    g(f"s_add_u32 {s_(S_KDMA)}, {s_(S_KDMA)}, %[ktile]")
    g(f"s_addc_u32 {s_(S_KDMA + 1)}, {s_(S_KDMA + 1)}, 0")
    g(f"s_cmp_le_u32 %[nkt], 1")
    g(f"s_cbranch_scc1 {no_k1}")
    g(f"s_cmp_eq_u32 %[nkt], 2")
    g(f"s_cselect_b32 {s_(S_ROWLIM)}, {s_(S_VALID)}, {BN}")
    g(f"s_sub_u32 {s_(S_ROWLIM)}, {s_(S_ROWLIM)}, 1")
    for i in range(4):
        kdma(g, i)
    g.label(no_k1)
    g(f"s_mov_b32 {s_(S_T3)}, {s_(S_VST + 1)}")
    g(f"s_mov_b32 {s_(S_VST + 1)}, {s_(S_VST)}")
    for i in range(4):
        vdma(g, i)
    g(f"s_mov_b32 {s_(S_VST + 1)}, {s_(S_T3)}")
    g(f"s_add_u32 {s_(S_VDMA)}, {s_(S_VDMA)}, {BN * 2}")
    g(f"s_addc_u32 {s_(S_VDMA + 1)}, {s_(S_VDMA + 1)}, 0")
    g(f"s_add_u32 {s_(S_KDMA)}, {s_(S_KDMA)}, %[ktile]")
    g(f"s_addc_u32 {s_(S_KDMA + 1)}, {s_(S_KDMA + 1)}, 0")
    # S(0) = K(0) Q^T into set A (K addresses of stage 0)
    for i in range(4):
        g(f"v_add_u32 {vr(KADDR + i)}, {s_(S_KST)}, %[kbase{i}]")
    g.lds = []
    k_read(g, 0, 0)
    k_read(g, 0, 1)
    k_read(g, 1, 0)
    k_read(g, 1, 1)
    s_phase(g, 0, items=None, dma=None, vreads_after=False)
    g.nops(20)
    # m = exact max of tile 0
    for qb in range(2):
        row_max_to(g, 0, qb, DTMP + 1, DTMP + 2)
        g(f"v_sub_f32 {vr(NEGM + qb)}, 0, {vr(DTMP + 1)}")
    g("s_waitcnt vmcnt(0)")
    g("s_barrier")
    # stage roles for tile 0: K(1) is read from stage 1 and K(2) goes to stage 0;
    # the first reads of K(1) are issued here, as a tile expects
    g(f"s_mov_b32 {s_(S_T0)}, {s_(S_KST)}")
    g(f"s_mov_b32 {s_(S_KST)}, {s_(S_KST + 1)}")
    g(f"s_mov_b32 {s_(S_KST + 1)}, {s_(S_T0)}")
    for i in range(4):
        g(f"v_add_u32 {vr(KADDR + i)}, {s_(S_KST)}, %[kbase{i}]")
    g.lds = []
    k_read(g, 0, 0)
    k_read(g, 0, 1)
    k_read(g, 1, 0)
    k_read(g, 1, 1)


def epilogue(g):
    """l total over both half-waves, O / l to bf16, stores; lse when asked."""
    g.nops(20)
    for qb in range(2):
        lt, inv, t = DTMP + 0, DTMP + 1, DTMP + 2
        g(f"ds_bpermute_b32 {vr(t)}, %[xaddr], {vr(LRUN + qb)}")
        g("s_waitcnt lgkmcnt(0)")
        g(f"v_add_f32 {vr(lt)}, {vr(LRUN + qb)}, {vr(t)}")
        # inv = l > 0 ? 1 / l : 0  (IEEE division sequence)
        g(f"v_div_scale_f32 {vr(TMP)}, {sp(S_CMP)}, {vr(lt)}, {vr(lt)}, 1.0")
        g(f"v_rcp_f32 {vr(TMP + 1)}, {vr(TMP)}")
        g("s_nop 0")
        g(f"v_fma_f32 {vr(TMP + 2)}, -{vr(TMP)}, {vr(TMP + 1)}, 1.0")
        g(f"v_fmac_f32 {vr(TMP + 1)}, {vr(TMP + 2)}, {vr(TMP + 1)}")
        g(f"v_div_scale_f32 {vr(TMP + 3)}, vcc, 1.0, {vr(lt)}, 1.0")
        g(f"v_mul_f32 {vr(TMP + 4)}, {vr(TMP + 3)}, {vr(TMP + 1)}")
        g(f"v_fma_f32 {vr(TMP + 5)}, -{vr(TMP)}, {vr(TMP + 4)}, {vr(TMP + 3)}")
        g(f"v_fmac_f32 {vr(TMP + 4)}, {vr(TMP + 5)}, {vr(TMP + 1)}")
        g(f"v_fma_f32 {vr(TMP + 3)}, -{vr(TMP)}, {vr(TMP + 4)}, {vr(TMP + 3)}")
        g(f"v_div_fmas_f32 {vr(TMP + 3)}, {vr(TMP + 3)}, {vr(TMP + 1)}, {vr(TMP + 4)}")
        g(f"v_div_fixup_f32 {vr(inv)}, {vr(TMP + 3)}, {vr(lt)}, 1.0")
        g(f"v_cmp_lt_f32 vcc, 0, {vr(lt)}")
        g(f"v_cndmask_b32 {vr(inv)}, 0, {vr(inv)}, vcc")
        # rows of this query block that exist: exec = (qrow < q_end)
        skip = g.new_label("nostore")
        g(f"s_mov_b64 {sp(S_EXEC)}, exec")
        g(f"v_cmp_gt_i32 vcc, %[qend], %[qrow{qb}]")
        g("s_and_b64 exec, exec, vcc")
        g(f"s_cbranch_execz {skip}")
        # output row address: obase + qrow * ldob + hh * 8 bytes (+ (d*32 + g*8) * 2)
        addr = S_SET[0]  # v[0:1] (S set A is dead here)
        g(f"v_mad_u64_u32 {vr(addr, 2)}, {sp(S_CMP)}, %[qrow{qb}], %[ldob], 0")
        g(f"v_add_co_u32 {vr(addr)}, vcc, %[obase_lo], {vr(addr)}")
        g(f"v_mov_b32 {vr(addr + 2)}, %[obase_hi]")
        g(f"v_addc_co_u32 {vr(addr + 1)}, vcc, {vr(addr + 2)}, {vr(addr + 1)}, vcc")
        g(f"v_add_co_u32 {vr(addr)}, vcc, %[hh8], {vr(addr)}")
        g(f"v_addc_co_u32 {vr(addr + 1)}, vcc, 0, {vr(addr + 1)}, vcc")
        for d in range(4):
            for gg in range(4):
                w0, w1 = 4, 5
                base = o_reg(qb, d) + gg * 4
                for k in range(4):
                    g(f"v_accvgpr_read_b32 {vr(8 + k)}, {ar(base + k)}")
                for k in range(4):
                    g(f"v_mul_f32 {vr(8 + k)}, {vr(8 + k)}, {vr(inv)}")
                g(f"v_cvt_pk_bf16_f32 {vr(w0)}, {vr(8)}, {vr(9)}")
                g(f"v_cvt_pk_bf16_f32 {vr(w1)}, {vr(10)}, {vr(11)}")
                g(f"global_store_dwordx2 {vr(addr, 2)}, {vr(w0, 2)}, off offset:{(d * 32 + gg * 8) * 2}")
        # lse = (m + log2 l) * ln 2 for lanes of the first half-wave, when asked
        g(f"s_cmp_eq_u32 %[has_lse], 0")
        g(f"s_cbranch_scc1 {skip}")
        g(f"v_cmp_gt_u32 vcc, 32, %[lane]")
        g("s_and_b64 exec, exec, vcc")
        g(f"s_cbranch_execz {skip}")
        g(f"v_log_f32 {vr(12)}, {vr(lt)}")
        g("s_nop 0")
        g(f"v_sub_f32 {vr(12)}, {vr(12)}, {vr(NEGM + qb)}")
        g(f"v_mul_f32 {vr(12)}, 0x3f317218, {vr(12)}")
        g(f"v_cmp_lt_f32 vcc, 0, {vr(lt)}")
        g(f"v_mov_b32 {vr(14)}, 0xff800000")
        g(f"v_cndmask_b32 {vr(12)}, {vr(14)}, {vr(12)}, vcc")
        g(f"v_lshlrev_b32 {vr(13)}, 2, %[qrow{qb}]")
        g(f"global_store_dword {vr(13)}, {vr(12)}, %[lsebase]")
        g.label(skip)
        g(f"s_mov_b64 exec, {sp(S_EXEC)}")


def generate():
    g = Gen()
    prologue(g)
    last_a = g.new_label("lastA")
    last_b = g.new_label("lastB")
    loop = g.new_label("loop")
    fin = g.new_label("fin")
    # P(0) keys 0..31 against the exact max (no check needed), only when a
    # steady tile follows
    g(f"s_cmp_le_u32 %[nkt], 1")
    g(f"s_cbranch_scc1 {last_a}")
    items = make_items(g, pair_list(0), 0, 0, RS0)
    g.nops(4)
    for it in items:
        it()
    g.label(loop)
    ra, ba = tile(g, 0)
    g(f"s_add_u32 {s_(S_T0)}, {s_(S_KT)}, 1")
    g(f"s_cmp_ge_u32 {s_(S_T0)}, %[nkt]")
    g(f"s_cbranch_scc1 {last_b}")
    rb, bb = tile(g, 1)
    g(f"s_add_u32 {s_(S_T0)}, {s_(S_KT)}, 1")
    g(f"s_cmp_ge_u32 {s_(S_T0)}, %[nkt]")
    g(f"s_cbranch_scc1 {last_a}")
    g(f"s_branch {loop}")
    rescale_block(g, 0, ra, ba)
    rescale_block(g, 1, rb, bb)
    g.label(last_a)
    last_tile(g, 0)
    g(f"s_branch {fin}")
    g.label(last_b)
    last_tile(g, 1)
    g.label(fin)
    epilogue(g)
    return g.lines


def main(argv):
    here = os.path.dirname(os.path.abspath(__file__))
    args = [a for a in argv[1:] if not a.startswith("--")]
    for a in argv[1:]:
        if a.startswith("--p2wait="):
            OPTS["p2wait"] = int(a.split("=", 1)[1])
        elif a == "--dma-block":
            OPTS["dma_slots"] = False
        elif a.startswith("--barrier-slot="):
            OPTS["barrier_slot"] = int(a.split("=", 1)[1])
    out = args[0] if args else os.path.join(here, "attn_d128_body.inc")
    lines = generate()
    with open(out, "w") as f:
        f.write("// Generated by gen_attn_d128.py -- the instruction body of flash_fwd_d128.\n")
        for line in lines:
            esc = line.replace("\\", "\\\\").replace('"', '\\"')
            f.write(f'"{esc}\\n"\n')
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
