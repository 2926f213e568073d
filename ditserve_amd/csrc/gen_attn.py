"""Generate the instruction body of the varlen flash-attention kernel
(attention.hip: flash_fwd_asm<HD>) as gfx950 assembly, for head dims 128 and 64.

Why generated assembly: the kernel runs one wave per SIMD with 64 queries per
wave, which needs about 460 registers per lane.  The compiler cannot place that
working set (its allocation spills or shuffles AGPR<->VGPR copies), so the
registers are assigned here by hand (head dim 128; at head dim 64 the O, Q, K
and Vt blocks halve and the VGPR map is the same):

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
  VGPR v208..v211  K DMA source offsets (switched to the clamped ones for the
                   last tile)
  VGPR v212..v215  temporaries
  AGPR a0..a127    O^T accumulators [qb][d] (16 each)
  AGPR a128..a191  Q fragments [qb][c] (4 each)
  AGPR a192..a215  K fragment ring: 3 chunks x 2 (kk)
  AGPR a216..a239  Vt fragment ring: 6 fragments
The LDS read addresses and DMA offsets that never change are compiler-placed
input operands; the K and Vt stages alternate with the tile parity, so the
stage is an immediate offset of each LDS read and DMA.

Per 64-key tile kt the wave (queries q0..q0+63 of one (segment, head)) runs
  phase 1: S(kt+1) = K(kt+1) Q^T    (32 MFMAs)  ||  P(kt) keys 32..63 (VALU)
  check:   lazy-rescale test on the row sums of P(kt)
  phase 2: O += Vt(kt) P(kt)        (32 MFMAs)  ||  P(kt+1) keys 0..31 (VALU)
with one VALU half-item per MFMA slot, K fragments read two chunks ahead and
Vt fragments four fragments ahead, and the next tiles' K and Vt streamed into
LDS by direct global->LDS DMA.  The arithmetic per score, the order of every
row sum and the rescale rule are those of the compiler-scheduled C++ kernel
this body replaced (8 waves of 32 queries), which it matched bitwise wherever
no rescale fired.

Hazards the hardware does not interlock are covered explicitly: an s_nop before
VALU reads of MFMA results and before MFMAs read AGPRs written by
v_accvgpr_write, an s_nop between an M0 write and the DMA that reads it.

Usage: python gen_attn.py [dir/any]  (writes attn_d128_body.inc, attn_d128p_body.inc,
attn_d64_body.inc, attn_d64p_body.inc, attn_d64j_body.inc and their
*_clobbers.h into that directory, default beside this file)
"""
import os
import sys

# ----------------------------------------------------------------------------
# register map (VGPRs: the same for both head dims)
S_SET = (0, 64)
P_SET = (128, 160)
VRING = 6        # Vt fragment ring (read four fragments ahead)
BN = 64


def configure(hd, pre=False, joint=False):
    """Head dim 128 or 64: NC 16-wide chunks of the head dim (K fragments per key
    half), DT 32-row d tiles of O^T, NF Vt fragments per tile (4 key groups x DT),
    ND DMA instructions per wave and operand per tile; AGPRs: O^T, then Q, the K
    ring (3 chunks x 2 key halves) and the Vt ring.

    pre: q arrives multiplied by softmax_scale * log2(e), and the first MFMA of
    every S accumulator starts from a block of 16 registers holding -m (one block
    per query block, v210..v241), so S is already q.k - m in log2 units and
    P = exp2(S) needs no per-score fma.  The VGPRs for the blocks come from a
    two-pair exp ring with the tile temporaries above it, no separate -m
    registers, and the per-lane operands used only outside the loop (Q and K DMA
    offsets, output rows, lane constants) passed in AGPRs.

    joint (with pre): a segment's rows are the rows of one segment of an "image"
    source followed by those of a "text" source (SD3.5's joint attention).  A key
    tile wholly in one source is DMA'd from that source's base with the usual
    lane offsets; the one tile per segment across the seam is DMA'd at the tile
    start in two lane-masked rounds (the slotted DMAs of that tile run with an
    empty exec mask).  Q rows are loaded through per-lane 64-bit addresses and
    output rows stored to the source they belong to.  Vt comes in the joint
    layout.  One query tile per work item."""
    global HD, NC, DT, NF, ND, KSTAGE_BYTES, VSTAGE_BYTES, O_A, Q_A, KF_A, VF_A, LAST_AGPR
    global PRE, TMP, RING, DTMP, RS0, RS1, NEGM, NEGB, LRUN, KOFF, LAST_VGPR, EPI_T, EPI_L, JOINT
    assert pre or not joint
    HD, PRE, JOINT = hd, pre, joint
    TMP = 192
    if pre:
        RING, DTMP = 2, 196
        RS0, RS1, LRUN, KOFF, NEGB, NEGM = 200, 202, 204, 206, 210, None
        LAST_VGPR = 241
        EPI_T, EPI_L = 64, 70          # epilogue temporaries in S set B (dead there)
    else:
        RING = 4                       # exp temporaries: a ring of four score pairs
        RS0, RS1, NEGM, LRUN, KOFF, DTMP, NEGB = 200, 202, 204, 206, 208, 212, None
        LAST_VGPR = 215
        EPI_T, EPI_L = TMP, DTMP
    NC, DT = hd // 16, hd // 32
    NF = 4 * DT
    ND = hd // 32
    KSTAGE_BYTES = VSTAGE_BYTES = BN * hd * 2
    O_A = 0
    Q_A = O_A + 2 * DT * 16
    KF_A = Q_A + 2 * NC * 4
    VF_A = KF_A + 3 * 2 * 4
    LAST_AGPR = VF_A + 4 * VRING - 1


configure(128)

# scalar registers owned by the body (all callee state lives in these)
S_KDMA = 60      # s[60:61] K DMA base (bytes) of tile min(kt+2, nkt-1)
S_VDMA = 62      # s[62:63] Vt DMA base (bytes) of tile kt+1
S_KW = 64        # s64 LDS K base + this wave's 1 KiB DMA slice
S_VW = 65        # s65 LDS Vt base + this wave's 1 KiB DMA slice
S_KT = 66        # s66 tile index kt
S_NKT1 = 67      # s67 nkt - 1
S_T0, S_T1 = 68, 69
S_CMP = 70       # s[70:71] compare mask
S_EXEC = 72      # s[72:73] saved exec
S_VALID = 74     # s74 valid keys of the last tile
S_THR = 75       # s75 the lazy-rescale threshold 256.0
S_QOFF = 76      # s76 query-row offset of the current pass (256 per pass)
S_NPASS = 77     # s77 passes left, this one included
S_KEXEC = 78     # s[78:79] joint: exec mask of the slotted K DMAs of this tile
S_KB2 = 80       # s[80:81] joint: the text source's K DMA base of the target tile
SGPRS = list(range(60, 78))
SGPRS_JOINT = list(range(60, 82))


def s_(n):
    return f"s{n}"


def negm(qb):
    """The register holding -m of query block qb (the first of its block when pre)."""
    return NEGB + 16 * qb if PRE else NEGM + qb


def opnd(g, name, tmp):
    """A per-lane operand as a VGPR operand string: when pre it arrives in an AGPR
    and is copied to VGPR tmp first."""
    if PRE:
        g(f"v_accvgpr_read_b32 {vr(tmp)}, %[{name}]")
        return vr(tmp)
    return f"%[{name}]"


def sp(n):
    return f"s[{n}:{n + 1}]"


def xaddr_to(g, dst, lane=None):
    """VGPR dst = the ds_bpermute byte address of lane ^ 32 (the other half-wave);
    lane: a VGPR already holding the lane index, else the operand."""
    src = lane if lane is not None else opnd(g, "lane", dst)
    g(f"v_xor_b32 {vr(dst)}, 32, {src}")
    g(f"v_lshlrev_b32 {vr(dst)}, 2, {vr(dst)}")
    return vr(dst)


def hh8_to(g, dst):
    """VGPR dst = 8 (lane / 32): this half-wave's key offset in a 16-key group."""
    g(f"v_lshrrev_b32 {vr(dst)}, 5, {opnd(g, 'lane', dst)}")
    g(f"v_lshlrev_b32 {vr(dst)}, 3, {vr(dst)}")
    return vr(dst)


def q_row_addr(g, row, a, t):
    """VGPRs a, a + 1 (a even) = the 64-bit address of this lane's 16 bytes of Q row `row`
    (VGPR, already clamped into the segment): qbase + row * ldq + 16 (lane / 32)
    bytes.  t: a free VGPR.  64-bit, so the packed Q may exceed 4 GiB."""
    g(f"v_mad_u64_u32 {vr(a, 2)}, {sp(S_CMP)}, {vr(row)}, %[ldqb], 0")
    g(f"v_add_co_u32 {vr(a)}, vcc, %[qbase_lo], {vr(a)}")
    g(f"v_mov_b32 {vr(t)}, %[qbase_hi]")
    g(f"v_addc_co_u32 {vr(a + 1)}, vcc, {vr(t)}, {vr(a + 1)}, vcc")
    g(f"v_lshrrev_b32 {vr(t)}, 5, {opnd(g, 'lane', t)}")
    g(f"v_lshlrev_b32 {vr(t)}, 4, {vr(t)}")
    g(f"v_add_co_u32 {vr(a)}, vcc, {vr(t)}, {vr(a)}")
    g(f"v_addc_co_u32 {vr(a + 1)}, vcc, 0, {vr(a + 1)}, vcc")


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
    return O_A + (qb * DT + d) * 16


def q_reg(qb, c):
    return Q_A + (qb * NC + c) * 4


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
    P, and the row sum rs += (p0 + p1).  The first pair of a query block starts
    the sum (rs = p0 + p1, the same value as 0 + (p0 + p1))."""
    qb, kk, j, e = pair
    t0 = TMP + 2 * (pi % RING)
    t1 = t0 + 1
    if half == 0:
        s0 = s_reg(s_set, qb, kk, j * 8 + 2 * e)
        if PRE:
            g(f"v_exp_f32 {vr(t0)}, {vr(s0)}")
            g(f"v_exp_f32 {vr(t1)}, {vr(s0 + 1)}")
        else:
            g(f"v_fma_f32 {vr(t0)}, {vr(s0)}, %[sc], {vr(NEGM + qb)}")
            g(f"v_fma_f32 {vr(t1)}, {vr(s0 + 1)}, %[sc], {vr(NEGM + qb)}")
            g(f"v_exp_f32 {vr(t0)}, {vr(t0)}")
            g(f"v_exp_f32 {vr(t1)}, {vr(t1)}")
    else:
        g(f"v_cvt_pk_bf16_f32 {vr(p_reg(p_set, qb, kk * 2 + j, e))}, {vr(t0)}, {vr(t1)}")
        if j == 0 and e == 0:
            g(f"v_add_f32 {vr(rs_base + qb)}, {vr(t0)}, {vr(t1)}")
        else:
            g(f"v_add_f32 {vr(t0)}, {vr(t0)}, {vr(t1)}")
            g(f"v_add_f32 {vr(rs_base + qb)}, {vr(rs_base + qb)}, {vr(t0)}")


# LDS DMA: M0 carries this wave's LDS destination (stage base + 1 KiB slice +
# 4 KiB per instruction); each lane moves 16 bytes.  The M0 write and the DMA
# that reads it are one instruction apart at least (one wait state).
def kdma_m0(g, i, stage):
    g(f"s_add_u32 m0, {s_(S_KW)}, {stage * KSTAGE_BYTES + i * 4096}")


def kdma_go(g, i):
    if JOINT:
        g(f"s_mov_b64 exec, {sp(S_KEXEC)}")
        g(f"global_load_lds_dwordx4 {vr(KOFF + i)}, {sp(S_KDMA)}")
        g("s_mov_b64 exec, -1")
    else:
        g(f"global_load_lds_dwordx4 {vr(KOFF + i)}, {sp(S_KDMA)}")


def joint_k_bases(g):
    """Joint: K DMA bases of target tile T = S_T0 in both sources (S_KDMA: image,
    S_KB2: text, each shifted so that lane offsets of tile rows apply) and S_T1 =
    image rows of the segment from the tile's first row on (len_img - 64 T)."""
    g(f"s_mul_i32 {s_(S_KDMA)}, {s_(S_T0)}, %[ktile]")
    g(f"s_mul_hi_u32 {s_(S_KDMA + 1)}, {s_(S_T0)}, %[ktile]")
    g(f"s_add_u32 {s_(S_KB2)}, {s_(S_KDMA)}, %[ktxt_lo]")
    g(f"s_addc_u32 {s_(S_KB2 + 1)}, {s_(S_KDMA + 1)}, %[ktxt_hi]")
    g(f"s_add_u32 {s_(S_KDMA)}, {s_(S_KDMA)}, %[kdma_lo]")
    g(f"s_addc_u32 {s_(S_KDMA + 1)}, {s_(S_KDMA + 1)}, %[kdma_hi]")
    g(f"s_lshl_b32 {s_(S_T1)}, {s_(S_T0)}, 6")
    g(f"s_sub_i32 {s_(S_T1)}, %[lena], {s_(S_T1)}")


def joint_k_dma_now(g, stage, tmp):
    """Joint: DMA target tile T = S_T0 (bases from joint_k_bases, KOFF already
    the clamped offsets if T is the last tile) into K stage `stage` now, in two
    lane-masked rounds: lanes whose row (clamped like their offset) is an image
    row, then the rest from the text source.  tmp: a free VGPR."""
    g(f"s_cmp_eq_u32 {s_(S_T0)}, {s_(S_NKT1)}")
    g(f"s_cselect_b32 {s_(S_CMP)}, {s_(S_VALID)}, {BN}")
    g(f"s_sub_u32 {s_(S_CMP)}, {s_(S_CMP)}, 1")
    for i in range(ND):
        g(f"v_accvgpr_read_b32 {vr(tmp)}, %[krow{i}]")
        g(f"v_min_u32 {vr(tmp)}, {s_(S_CMP)}, {vr(tmp)}")
        g(f"v_cmp_gt_i32 vcc, {s_(S_T1)}, {vr(tmp)}")
        kdma_m0(g, i, stage)
        g("s_mov_b64 exec, vcc")
        g(f"global_load_lds_dwordx4 {vr(KOFF + i)}, {sp(S_KDMA)}")
        g("s_not_b64 exec, vcc")
        g(f"global_load_lds_dwordx4 {vr(KOFF + i)}, {sp(S_KB2)}")
        g("s_mov_b64 exec, -1")


def vdma_m0(g, i, stage):
    g(f"s_add_u32 m0, {s_(S_VW)}, {stage * VSTAGE_BYTES + i * 4096}")


def vdma_go(g, i):
    g(f"global_load_lds_dwordx4 %[voff{i}], {sp(S_VDMA)}")


def kdma_block(g, stage):
    for i in range(ND):
        kdma_m0(g, i, stage)
        g("s_nop 0")
        kdma_go(g, i)


def vdma_block(g, stage):
    for i in range(ND):
        vdma_m0(g, i, stage)
        g("s_nop 0")
        vdma_go(g, i)


def clamp_koff(g, cmp):
    """K DMA offsets of the last tile (rows past the end read the last row) when
    the scalar compare `cmp` holds."""
    skip = g.new_label("noclamp")
    g(cmp)
    g(f"s_cbranch_scc0 {skip}")
    for i in range(ND):
        if PRE:
            g(f"v_accvgpr_read_b32 {vr(KOFF + i)}, %[koffl{i}]")
        else:
            g(f"v_mov_b32 {vr(KOFF + i)}, %[koffl{i}]")
    g.label(skip)


def k_read(g, chunk, kk, stage):
    """ds_read of K fragment (chunk, kk) of K stage `stage`."""
    off = stage * KSTAGE_BYTES + (chunk >> 2) * 8192 + kk * 4096
    g(f"ds_read_b128 {ar(kf_reg(chunk % 3, kk), 4)}, %[kaddr{chunk & 3}] offset:{off}")
    g.lds_issue(("k", chunk, kk))


def v_read(g, f, stage):
    grp, d = f // DT, f % DT
    g(f"ds_read_b128 {ar(vf_reg(f % VRING), 4)}, %[vaddr{grp}] offset:{stage * VSTAGE_BYTES + d * 4096}")
    g.lds_issue(("v", f))


def mfma_s(g, s_set, qb, kk, chunk, first=False):
    """first: the prologue's S(0), started from 0 also when pre (m not known yet)."""
    dst = s_reg(s_set, qb, kk)
    if chunk > 0:
        src_c = vr(dst, 16)
    else:
        src_c = vr(negm(qb), 16) if PRE and not first else "0"
    g(f"v_mfma_f32_32x32x16_bf16 {vr(dst, 16)}, {ar(kf_reg(chunk % 3, kk), 4)}, {ar(q_reg(qb, chunk), 4)}, {src_c}")


def mfma_o(g, p_set, qb, d, grp, ring):
    o = o_reg(qb, d)
    g(f"v_mfma_f32_32x32x16_bf16 {ar(o, 16)}, {ar(vf_reg(ring), 4)}, {vr(p_reg(p_set, qb, grp), 4)}, {ar(o, 16)}")


def s_phase(g, s_set, kstage, vstage=None, items=None, dma=None, first=False):
    """32 S MFMAs (into s_set) with K fragments of K stage kstage read two chunks
    ahead; the first two chunks' reads must already be issued.  vstage: issue the
    first four Vt reads of that stage after the last chunk's first MFMA.  items:
    one callable per slot; dma: (before, after) callables around the MFMA of the
    first slots."""
    slot = 0
    for c in range(NC):
        g.lds_wait(("k", c, 1))
        for kk in range(2):
            for qb in range(2):
                d = dma[slot] if dma is not None and slot < len(dma) else None
                if d:
                    d[0]()
                mfma_s(g, s_set, qb, kk, c, first)
                if kk == 0 and qb == 0 and c + 2 < NC:
                    k_read(g, c + 2, 0, kstage)
                    k_read(g, c + 2, 1, kstage)
                if kk == 0 and qb == 0 and c == NC - 1 and vstage is not None:
                    for f in range(4):
                        v_read(g, f, vstage)
                if d:
                    d[1]()
                if items is not None:
                    items[slot]()
                slot += 1


def o_phase(g, p_set, vstage, items=None):
    """32 PV MFMAs with Vt fragments of stage vstage four ahead (the first four
    already issued), waited for in pairs."""
    slot = 0
    for f in range(NF):
        grp, d = f // DT, f % DT
        for qb in range(2):
            if qb == 0 and f % 2 == 0:
                g.lds_wait(("v", f + 1))
            mfma_o(g, p_set, qb, d, grp, f % VRING)
            if qb == 0 and f + 4 < NF:
                v_read(g, f + 4, vstage)
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


def row_max_to(g, s_set, qb, dst, tmp, atmp):
    """dst = max over this lane's 32 scores of query block qb (both half-waves
    combined), times the softmax scale (log2 units; pre: the scores already are).
    atmp: a VGPR for the exchange address when it arrives in an AGPR."""
    base = s_reg(s_set, qb, 0)
    g(f"v_max3_f32 {vr(dst)}, {vr(base)}, {vr(base + 16)}, {vr(base + 1)}")
    for v in range(1, 16):
        a, b = base + v, base + 16 + v
        if v == 1:
            g(f"v_max_f32 {vr(dst)}, {vr(dst)}, {vr(b)}")
        else:
            g(f"v_max3_f32 {vr(dst)}, {vr(dst)}, {vr(a)}, {vr(b)}")
    xa = xaddr_to(g, atmp)
    g(f"ds_bpermute_b32 {vr(tmp)}, {xa}, {vr(dst)}")
    g("s_waitcnt lgkmcnt(0)")
    g(f"v_max_f32 {vr(dst)}, {vr(dst)}, {vr(tmp)}")
    if not PRE:
        g(f"v_mul_f32 {vr(dst)}, %[sc], {vr(dst)}")


def scale_o(g, qb, alpha):
    for d in range(DT):
        for v in range(16):
            a = o_reg(qb, d) + v
            g(f"v_accvgpr_read_b32 {vr(DTMP)}, {ar(a)}")
            g(f"v_mul_f32 {vr(DTMP)}, {vr(DTMP)}, {vr(alpha)}")
            g(f"v_accvgpr_write_b32 {ar(a)}, {vr(DTMP)}")


def softmax_tile(g, s_set, p_set, qb, kks, rs_dst, masked=False):
    """Recompute P for the given key halves of query block qb from the raw scores
    and the running m (pre: from S = q.k - m); rs_dst += sum (masked: keys >=
    valid excluded)."""
    hh8 = hh8_to(g, TMP + 3) if masked else None
    for kk in kks:
        for j in range(2):
            for e in range(4):
                s0 = s_reg(s_set, qb, kk, j * 8 + 2 * e)
                t0, t1 = TMP, TMP + 1
                if PRE:
                    g(f"v_exp_f32 {vr(t0)}, {vr(s0)}")
                    g(f"v_exp_f32 {vr(t1)}, {vr(s0 + 1)}")
                else:
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
                        g(f"v_cmp_gt_i32 vcc, {s_(S_T0)}, {hh8}")
                        g(f"v_cndmask_b32 {vr(t)}, 0, {vr(t)}, vcc")
                g(f"v_add_f32 {vr(t0)}, {vr(t0)}, {vr(t1)}")
                g(f"v_add_f32 {vr(rs_dst + qb)}, {vr(rs_dst + qb)}, {vr(t0)}")


def exact_rescale(g, s_set, p_set, kks, masked=False, live_next=None):
    """The C++ rescale: m_new = max(m, row max of the tile's scores), O and l
    scaled by exp2(m - m_new), P of the tile recomputed against m_new into rs0.
    (rs1 is cleared.)  Pre: the scores are relative to m_old, so m_new = max(m_old,
    row max + m_old); the tile's S and the next tile's (S set live_next, started
    from the old -m block) move by -(m_new - m_old) and the block becomes -m_new."""
    g.nops(20)  # O accumulators read below: MFMA results must have landed
    for qb in range(2):
        mx, tmp, alpha = DTMP + 1, DTMP + 2, DTMP + 3
        row_max_to(g, s_set, qb, mx, tmp, alpha)
        if PRE:
            nb = negm(qb)
            g(f"v_sub_f32 {vr(tmp)}, 0, {vr(nb)}")            # m_old
            g(f"v_add_f32 {vr(mx)}, {vr(mx)}, {vr(tmp)}")     # row max + m_old
            g(f"v_max_f32 {vr(mx)}, {vr(tmp)}, {vr(mx)}")     # m_new
            g(f"v_sub_f32 {vr(alpha)}, {vr(tmp)}, {vr(mx)}")
            g(f"v_exp_f32 {vr(alpha)}, {vr(alpha)}")
            g(f"v_sub_f32 {vr(tmp)}, {vr(mx)}, {vr(tmp)}")    # m_new - m_old
            g(f"v_sub_f32 {vr(mx)}, 0, {vr(mx)}")
            for v in range(16):
                g(f"v_mov_b32 {vr(nb + v)}, {vr(mx)}")
            for st in (s_set,) if live_next is None else (s_set, live_next):
                for kk in (kks if st == s_set else (0, 1)):
                    for v in range(16):
                        r = s_reg(st, qb, kk, v)
                        g(f"v_sub_f32 {vr(r)}, {vr(r)}, {vr(tmp)}")
        else:
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
    g.nops(5 if PRE else 3)  # v_accvgpr_write (and the -m block writes) -> MFMA srcC


def tile(g, a):
    """One steady tile kt (kt % 2 == a): scores of tile kt in S set a, S(kt+1)
    computed into set b = 1 - a.  Entered with the reads of K(kt+1) chunks 0 and
    1 already issued.

    LDS stages are fixed by parity: K(kt+1) is read from K stage b while K(tile
    min(kt+2, nkt-1)) is DMA'd into K stage a (K(kt) is read by no wave any
    more); Vt(kt) is read from Vt stage a while Vt(kt+1) is DMA'd into stage b.
    The workgroup barrier at the end of the tile publishes both DMAs."""
    b = 1 - a
    after_check = g.new_label("checked")
    resc = g.new_label("rescale")
    g.lds = [("k", 0, 0), ("k", 0, 1), ("k", 1, 0), ("k", 1, 1)]
    # K DMA source of tile min(kt+2, nkt-1); the last tile's rows past the end clamp
    g(f"s_add_u32 {s_(S_T0)}, {s_(S_KT)}, 2")
    g(f"s_min_u32 {s_(S_T0)}, {s_(S_T0)}, {s_(S_NKT1)}")
    if JOINT:
        clamp_koff(g, f"s_cmp_eq_u32 {s_(S_T0)}, {s_(S_NKT1)}")
        joint_k_bases(g)
        # wholly image: slotted DMAs from the image base; wholly text: from the
        # text base; across the seam: DMA'd here, slotted DMAs masked off
        kdone = g.new_label("kbase")
        g(f"s_mov_b64 {sp(S_KEXEC)}, -1")
        g(f"s_cmp_ge_i32 {s_(S_T1)}, {BN}")
        g(f"s_cbranch_scc1 {kdone}")
        g(f"s_mov_b64 {sp(S_KDMA)}, {sp(S_KB2)}")
        g(f"s_cmp_le_i32 {s_(S_T1)}, 0")
        g(f"s_cbranch_scc1 {kdone}")
        g(f"s_mov_b64 {sp(S_KEXEC)}, 0")
        joint_k_bases(g)
        joint_k_dma_now(g, a, S_SET[b])
        g.label(kdone)
    else:
        g(f"s_mul_i32 {s_(S_KDMA)}, {s_(S_T0)}, %[ktile]")
        g(f"s_mul_hi_u32 {s_(S_KDMA + 1)}, {s_(S_T0)}, %[ktile]")
        g(f"s_add_u32 {s_(S_KDMA)}, {s_(S_KDMA)}, %[kdma_lo]")
        g(f"s_addc_u32 {s_(S_KDMA + 1)}, {s_(S_KDMA + 1)}, %[kdma_hi]")
        clamp_koff(g, f"s_cmp_eq_u32 {s_(S_T0)}, {s_(S_NKT1)}")
    dmas = ([(lambda i=i: kdma_m0(g, i, a), lambda i=i: kdma_go(g, i)) for i in range(ND)] +
            [(lambda i=i: vdma_m0(g, i, b), lambda i=i: vdma_go(g, i)) for i in range(ND)])
    # phase 1: S(kt+1) into set b || P(kt) keys 32..63 from set a
    items = make_items(g, pair_list(1), a, a, RS1, slots=4 * NC)
    s_phase(g, b, kstage=b, vstage=a, items=items, dma=dmas)
    # lazy-rescale check on tile kt: rsum = rs0 + rs1 (per lane), flag !(rsum <= 256)
    for qb in range(2):
        g(f"v_add_f32 {vr(DTMP + qb)}, {vr(RS0 + qb)}, {vr(RS1 + qb)}")
    g(f"v_cmp_nge_f32 vcc, {s_(S_THR)}, {vr(DTMP)}")
    g(f"v_cmp_nge_f32_e64 {sp(S_CMP)}, {s_(S_THR)}, {vr(DTMP + 1)}")
    g(f"s_or_b64 vcc, vcc, {sp(S_CMP)}")
    g(f"s_cbranch_vccnz {resc}")
    g.label(after_check)
    for qb in range(2):
        g(f"v_add_f32 {vr(LRUN + qb)}, {vr(LRUN + qb)}, {vr(DTMP + qb)}")
    # phase 2: O += Vt(kt) P(kt) || P(kt+1) keys 0..31 from set b.  The wait
    # covers the VALU reads of the S(kt+1) results of the last MFMAs (already
    # three MFMAs old) and the MFMA reads of the P(kt) just packed.
    g.nops(2)
    items = make_items(g, pair_list(0), b, b, RS0, slots=2 * NF)
    o_phase(g, a, vstage=a, items=items)
    # publish this tile's DMA: own loads landed, then the workgroup barrier
    g("s_waitcnt vmcnt(0)")
    g("s_barrier")
    g(f"s_add_u32 {s_(S_VDMA)}, {s_(S_VDMA)}, {BN * 2}")
    g(f"s_addc_u32 {s_(S_VDMA + 1)}, {s_(S_VDMA + 1)}, 0")
    g(f"s_add_u32 {s_(S_KT)}, {s_(S_KT)}, 1")
    # the next tile's first K reads: K(kt+2), in stage a
    for c in range(2):
        k_read(g, c, 0, a)
        k_read(g, c, 1, a)
    return resc, after_check


def rescale_block(g, a, resc, back):
    """Out-of-line rescale of tile kt (scores still in set a, P(kt) in P set a);
    returns with the tile's row sums in DTMP like the common path."""
    g.label(resc)
    exact_rescale(g, a, a, (0, 1), live_next=1 - a)
    for qb in range(2):
        g(f"v_add_f32 {vr(DTMP + qb)}, {vr(RS0 + qb)}, {vr(RS1 + qb)}")
    g(f"s_branch {back}")


def last_tile_prefetch(g, a, nopf):
    """Under the last key tile of a pass with another pass to follow: that pass's
    Q loads, K(0)/K(1) DMAs and (Vt of this tile in stage 1) its Vt(0) DMA."""
    g(f"s_cmp_gt_u32 {s_(S_NPASS)}, 1")
    g(f"s_cbranch_scc0 {nopf}")
    tmp = S_SET[1 - a]  # S set of the next tile: free in the last tile
    g(f"s_add_u32 {s_(S_T0)}, {s_(S_QOFF)}, {BN * 4}")
    g(f"s_sub_u32 {s_(S_T1)}, %[qend], 1")
    for qb in range(2):
        ad = tmp + 4 * qb  # even: the address pair, then the row and a temporary
        qrow = opnd(g, f"qrow{qb}", ad + 2)
        g(f"v_add_u32 {vr(ad + 2)}, {s_(S_T0)}, {qrow}")
        g(f"v_min_i32 {vr(ad + 2)}, {s_(S_T1)}, {vr(ad + 2)}")
        q_row_addr(g, ad + 2, ad, ad + 3)
        for c in range(NC):
            g(f"global_load_dwordx4 {ar(q_reg(qb, c), 4)}, {vr(ad, 2)}, off offset:{c * 32}")
    first_k_dmas(g)
    if a == 1:
        first_vt_dma(g)


def last_tile(g, a):
    """The last key tile (kt % 2 == a, scores in set a): P of all 64 keys against
    m with keys past the segment end out of the row sums, the rescale test, then
    O += Vt P."""
    full = g.new_label("fullrs")
    done_rs = g.new_label("rsdone")
    resc = g.new_label("lastresc")
    checked = g.new_label("lastchecked")
    g.nops(20)
    g.lds_wait_all()
    # another pass follows: its Q (into the Q AGPRs, free since this tile has no
    # S MFMAs), K(0) and K(1) (no wave reads K any more: all passed the last
    # tile barrier), and, when this tile's Vt is in stage 1, Vt(0) into stage 0
    nopf = g.new_label("noprefetch")
    multi = not JOINT  # joint work items are one query tile (one pass)
    if multi:
        last_tile_prefetch(g, a, nopf)
    g.label(nopf)
    # a full last tile after a steady one: P keys 0..31 and their row sums were
    # made by that tile's phase 2, so only keys 32..63 are computed here and the
    # check is the steady tile's; otherwise P of all 64 keys is recomputed
    recompute = g.new_label("lastrecompute")
    common = g.new_label("lastpv")
    reuse_back = g.new_label("lastreuseback")
    g(f"s_cmp_eq_u32 {s_(S_VALID)}, {BN}")
    g(f"s_cbranch_scc0 {recompute}")
    g(f"s_cmp_eq_u32 {s_(S_NKT1)}, 0")
    g(f"s_cbranch_scc1 {recompute}")
    for it in make_items(g, pair_list(1), a, a, RS1):
        it()
    for qb in range(2):
        g(f"v_add_f32 {vr(DTMP + qb)}, {vr(RS0 + qb)}, {vr(RS1 + qb)}")
    g(f"v_cmp_nge_f32 vcc, {s_(S_THR)}, {vr(DTMP)}")
    g(f"v_cmp_nge_f32_e64 {sp(S_CMP)}, {s_(S_THR)}, {vr(DTMP + 1)}")
    g(f"s_or_b64 vcc, vcc, {sp(S_CMP)}")
    g(f"s_cbranch_vccz {reuse_back}")
    exact_rescale(g, a, a, (0, 1))
    for qb in range(2):
        g(f"v_add_f32 {vr(DTMP + qb)}, {vr(RS0 + qb)}, {vr(RS1 + qb)}")
    g.label(reuse_back)
    for qb in range(2):
        g(f"v_add_f32 {vr(LRUN + qb)}, {vr(LRUN + qb)}, {vr(DTMP + qb)}")
    g(f"s_branch {common}")
    g.label(recompute)
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
    g(f"v_cmp_nge_f32 vcc, {s_(S_THR)}, {vr(RS0)}")
    g(f"v_cmp_nge_f32_e64 {sp(S_CMP)}, {s_(S_THR)}, {vr(RS0 + 1)}")
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
    g.label(common)
    g("s_nop 2")
    for f in range(4):
        v_read(g, f, a)
    o_phase(g, a, vstage=a, items=None)
    # another pass: its loads landed and published, this tile's Vt reads done
    # in every wave; then Vt(0) into stage 0 if this tile used it
    if multi:
        nxt = g.new_label("lastdone")
        g(f"s_cmp_gt_u32 {s_(S_NPASS)}, 1")
        g(f"s_cbranch_scc0 {nxt}")
        g("s_waitcnt vmcnt(0)")
        g("s_barrier")
        if a == 0:
            first_vt_dma(g)
        g.label(nxt)


def first_k_dmas(g):
    """DMA K(0) into K stage 0 and K(1) into stage 1 (K(0) again when there is
    one tile), with the clamped offsets for whichever is the last tile."""
    if JOINT:
        for i in range(ND):
            g(f"v_accvgpr_read_b32 {vr(KOFF + i)}, %[koff{i}]")
        for t in range(2):
            g(f"s_min_u32 {s_(S_T0)}, {t}, {s_(S_NKT1)}")
            clamp_koff(g, f"s_cmp_eq_u32 {s_(S_T0)}, {s_(S_NKT1)}")
            joint_k_bases(g)
            joint_k_dma_now(g, t, S_SET[1])
        return
    for i in range(ND):
        if PRE:
            g(f"v_accvgpr_read_b32 {vr(KOFF + i)}, %[koff{i}]")
        else:
            g(f"v_mov_b32 {vr(KOFF + i)}, %[koff{i}]")
    g(f"s_mov_b32 {s_(S_KDMA)}, %[kdma_lo]")
    g(f"s_mov_b32 {s_(S_KDMA + 1)}, %[kdma_hi]")
    clamp_koff(g, f"s_cmp_eq_u32 {s_(S_NKT1)}, 0")
    kdma_block(g, 0)
    g(f"s_cmp_eq_u32 {s_(S_NKT1)}, 0")
    g(f"s_cselect_b32 {s_(S_T0)}, 0, %[ktile]")
    g(f"s_add_u32 {s_(S_KDMA)}, {s_(S_KDMA)}, {s_(S_T0)}")
    g(f"s_addc_u32 {s_(S_KDMA + 1)}, {s_(S_KDMA + 1)}, 0")
    clamp_koff(g, f"s_cmp_le_u32 {s_(S_NKT1)}, 1")
    kdma_block(g, 1)


def first_vt_dma(g):
    """DMA Vt(0) into Vt stage 0; the Vt DMA base then points at tile 1."""
    g(f"s_mov_b32 {s_(S_VDMA)}, %[vdma_lo]")
    g(f"s_mov_b32 {s_(S_VDMA + 1)}, %[vdma_hi]")
    vdma_block(g, 0)
    g(f"s_add_u32 {s_(S_VDMA)}, {s_(S_VDMA)}, {BN * 2}")
    g(f"s_addc_u32 {s_(S_VDMA + 1)}, {s_(S_VDMA + 1)}, 0")


def prologue(g, empty):
    """The first pass's loads.  empty: the label of the no-keys path (O = 0,
    l = 0: the epilogue then stores zero rows and lse = -inf)."""
    # scalar state
    g(f"s_mov_b32 {s_(S_QOFF)}, 0")
    g(f"s_mov_b32 {s_(S_NPASS)}, %[npass]")
    g(f"s_add_u32 {s_(S_KW)}, %[lds_k], %[wave1k]")
    g(f"s_add_u32 {s_(S_VW)}, %[lds_v], %[wave1k]")
    g(f"s_sub_u32 {s_(S_NKT1)}, %[nkt], 1")
    g(f"s_mov_b32 {s_(S_VALID)}, %[valid_last]")
    g(f"s_mov_b32 {s_(S_THR)}, 0x43800000")
    g("s_cmp_eq_u32 %[nkt], 0")
    g(f"s_cbranch_scc1 {empty}")
    # Q fragments straight into AGPRs, then the DMAs of K(0) (K stage 0), K(1)
    # (K stage 1; K(0) again when there is one tile) and Vt(0) (Vt stage 0), all
    # before the first wait so that their latencies overlap
    if PRE:
        g("s_nop 4")  # the AGPR operands were written just before the body
    for qb in range(2):
        if JOINT:  # per-lane 64-bit row address in its source
            qa = S_SET[0] + 2 * qb
            g(f"v_accvgpr_read_b32 {vr(qa)}, %[qa{qb}lo]")
            g(f"v_accvgpr_read_b32 {vr(qa + 1)}, %[qa{qb}hi]")
            for c in range(NC):
                g(f"global_load_dwordx4 {ar(q_reg(qb, c), 4)}, {vr(qa, 2)}, off offset:{c * 32}")
            continue
        # this lane's row, the segment's last row for the rows past its end
        ad = S_SET[0] + 4 * qb  # even: the address pair, then the row and a temporary
        g(f"s_sub_u32 {s_(S_T1)}, %[qend], 1")
        qrow = opnd(g, f"qrow{qb}", ad + 2)
        g(f"v_min_i32 {vr(ad + 2)}, {s_(S_T1)}, {qrow}")
        q_row_addr(g, ad + 2, ad, ad + 3)
        for c in range(NC):
            g(f"global_load_dwordx4 {ar(q_reg(qb, c), 4)}, {vr(ad, 2)}, off offset:{c * 32}")
    first_k_dmas(g)
    first_vt_dma(g)
    # O = 0, l = 0 while the loads fly
    clear_state(g)
    # Q and K(0) landed (the DMAs of K(1) and Vt(0) may still fly), K(0) published
    g(f"s_waitcnt vmcnt({2 * ND})")
    g("s_barrier")


def clear_state(g):
    """O = 0, l = 0, row sums 0, tile 0."""
    for i in range(2 * DT * 16):
        g(f"v_accvgpr_write_b32 {ar(O_A + i)}, 0")
    for qb in range(2):
        g(f"v_mov_b32 {vr(LRUN + qb)}, 0")
        g(f"v_mov_b32 {vr(RS0 + qb)}, 0")
        g(f"v_mov_b32 {vr(RS1 + qb)}, 0")
    g(f"s_mov_b32 {s_(S_KT)}, 0")


def pass_start(g):
    """S(0) of a pass (its Q, K(0) landed and published), the exact max of tile
    0, then the wait for K(1) and Vt(0)."""
    # S(0) = K(0) Q^T into set A
    g.lds = []
    for c in range(2):
        k_read(g, c, 0, 0)
        k_read(g, c, 1, 0)
    s_phase(g, 0, kstage=0, first=True)
    g.nops(20)
    # m = exact max of tile 0 (pre: S(0) -= m, and the -m blocks)
    for qb in range(2):
        row_max_to(g, 0, qb, DTMP + 1, DTMP + 2, DTMP + 3)
        if PRE:
            for kk in range(2):
                for v in range(16):
                    r = s_reg(0, qb, kk, v)
                    g(f"v_sub_f32 {vr(r)}, {vr(r)}, {vr(DTMP + 1)}")
            g(f"v_sub_f32 {vr(DTMP + 1)}, 0, {vr(DTMP + 1)}")
            for v in range(16):
                g(f"v_mov_b32 {vr(negm(qb) + v)}, {vr(DTMP + 1)}")
        else:
            g(f"v_sub_f32 {vr(NEGM + qb)}, 0, {vr(DTMP + 1)}")
    g("s_waitcnt vmcnt(0)")
    g("s_barrier")
    # tile 0 reads K(1) from K stage 1; its first reads are issued here
    g.lds = []
    for c in range(2):
        k_read(g, c, 0, 1)
        k_read(g, c, 1, 1)


def epilogue(g, negm_of=None):
    """l total over both half-waves, O / l to bf16, stores; lse when asked
    (negm_of(qb): the register holding -m of query block qb, default negm).

    Each 32-query block goes through this wave's LDS staging rows (pitch HD * 2 +
    8 bytes, query q at row q) so that the global stores write whole row
    segments: a lane owns 4 consecutive dims of one query in the accumulators,
    but stores 16 bytes of one row, HD / 8 lanes per row.  The stores are
    non-temporal: nothing in the kernel reads the output again."""
    g.nops(20)
    T = EPI_T
    # temporaries from register EB on: S set B past the EPI registers (dead in
    # every last tile; S set A may hold the next pass's scores), or S set A for
    # joint attention (one pass, and its addressing needs more registers)
    EB = 0 if JOINT else 76
    negm_of = negm_of or negm
    pitch = HD * 2 + 8
    lpr = HD // 8                  # lanes per output row (16 bytes each)
    rpr = 64 // lpr                # rows per store instruction
    addr, wa, ra, t0, left, ohi = EB, EB + 2, EB + 3, EB + 49, EB + 48, EB + 50
    data = EB + 16                 # read-back rows (4 per read)
    lane = opnd(g, "lane", EPI_L + 5)
    # LDS write address: row lane % 32, + 8 bytes for the upper half-wave;
    # read address: row lane / lpr, 16-byte column lane % lpr
    g(f"v_and_b32 {vr(t0)}, 31, {lane}")
    g(f"v_mul_u32_u24 {vr(wa)}, {pitch}, {vr(t0)}")
    g(f"v_lshrrev_b32 {vr(t0)}, 5, {lane}")
    g(f"v_lshl_add_u32 {vr(wa)}, {vr(t0)}, 3, {vr(wa)}")
    g(f"v_add_u32 {vr(wa)}, %[lds_o], {vr(wa)}")
    g(f"v_lshrrev_b32 {vr(t0)}, {lpr.bit_length() - 1}, {lane}")
    g(f"v_mul_u32_u24 {vr(ra)}, {pitch}, {vr(t0)}")
    g(f"v_and_b32 {vr(t0)}, {lpr - 1}, {lane}")
    g(f"v_lshl_add_u32 {vr(ra)}, {vr(t0)}, 4, {vr(ra)}")
    g(f"v_add_u32 {vr(ra)}, %[lds_o], {vr(ra)}")
    g(f"s_lshl_b32 {s_(S_T1)}, %[ldob], {rpr.bit_length() - 1}")   # rpr rows of output
    for qb in range(2):
        lt, inv, t = EPI_L + 0, EPI_L + 1, EPI_L + 2
        xa = xaddr_to(g, EPI_L + 3, lane)
        qrow = vr(EB + 51)  # this lane's query row in this pass
        g(f"v_add_u32 {qrow}, {s_(S_QOFF)}, {opnd(g, f'qrow{qb}', EPI_L + 4)}")
        g(f"ds_bpermute_b32 {vr(t)}, {xa}, {vr(LRUN + qb)}")
        g("s_waitcnt lgkmcnt(0)")
        g(f"v_add_f32 {vr(lt)}, {vr(LRUN + qb)}, {vr(t)}")
        # inv = l > 0 ? 1 / l : 0  (IEEE division sequence)
        g(f"v_div_scale_f32 {vr(T)}, {sp(S_CMP)}, {vr(lt)}, {vr(lt)}, 1.0")
        g(f"v_rcp_f32 {vr(T + 1)}, {vr(T)}")
        g("s_nop 0")
        g(f"v_fma_f32 {vr(T + 2)}, -{vr(T)}, {vr(T + 1)}, 1.0")
        g(f"v_fmac_f32 {vr(T + 1)}, {vr(T + 2)}, {vr(T + 1)}")
        g(f"v_div_scale_f32 {vr(T + 3)}, vcc, 1.0, {vr(lt)}, 1.0")
        g(f"v_mul_f32 {vr(T + 4)}, {vr(T + 3)}, {vr(T + 1)}")
        g(f"v_fma_f32 {vr(T + 5)}, -{vr(T)}, {vr(T + 4)}, {vr(T + 3)}")
        g(f"v_fmac_f32 {vr(T + 4)}, {vr(T + 5)}, {vr(T + 1)}")
        g(f"v_fma_f32 {vr(T + 3)}, -{vr(T)}, {vr(T + 4)}, {vr(T + 3)}")
        g(f"v_div_fmas_f32 {vr(T + 3)}, {vr(T + 3)}, {vr(T + 1)}, {vr(T + 4)}")
        g(f"v_div_fixup_f32 {vr(inv)}, {vr(T + 3)}, {vr(lt)}, 1.0")
        g(f"v_cmp_lt_f32 vcc, 0, {vr(lt)}")
        g(f"v_cndmask_b32 {vr(inv)}, 0, {vr(inv)}, vcc")
        # O / l -> bf16 into the staging rows (every lane; rows past the end are
        # written but never stored)
        for d in range(DT):
            for gg in range(4):
                w0, w1 = EB + 4, EB + 5
                base = o_reg(qb, d) + gg * 4
                for k in range(4):
                    g(f"v_accvgpr_read_b32 {vr(EB + 8 + k)}, {ar(base + k)}")
                for k in range(4):
                    g(f"v_mul_f32 {vr(EB + 8 + k)}, {vr(EB + 8 + k)}, {vr(inv)}")
                g(f"v_cvt_pk_bf16_f32 {vr(w0)}, {vr(EB + 8)}, {vr(EB + 9)}")
                g(f"v_cvt_pk_bf16_f32 {vr(w1)}, {vr(EB + 10)}, {vr(EB + 11)}")
                g(f"ds_write_b64 {vr(wa)}, {vr(w0, 2)} offset:{(d * 32 + gg * 8) * 2}")
        g("s_waitcnt lgkmcnt(0)")
        for i in range(32 // rpr):
            g(f"ds_read_b128 {vr(data + 4 * i, 4)}, {vr(ra)} offset:{i * rpr * pitch}")
        # this lane's first output row (block start + lane / lpr), rows left in
        # the segment, and its address: obase + row * ldob + (lane % lpr) * 16
        g(f"v_and_b32 {vr(t0)}, 31, {lane}")
        g(f"v_sub_u32 {vr(left)}, {qrow}, {vr(t0)}")
        g(f"v_lshrrev_b32 {vr(t0)}, {lpr.bit_length() - 1}, {lane}")
        g(f"v_add_u32 {vr(left)}, {vr(left)}, {vr(t0)}")
        if JOINT:
            # row j of the segment (j0 + i * rpr for store i) goes to the image
            # output while j < len_img, else to the text output; jbase[01] hold
            # the two sources' segment bases (shifted by len_img for text) plus
            # this lane's 16-byte column
            j0, ib, tb = EB + 52, EB + 53, EB + 55
            g(f"v_subrev_u32 {vr(j0)}, %[qseg], {vr(left)}")
            g(f"v_and_b32 {vr(t0)}, {lpr - 1}, {lane}")
            g(f"v_lshlrev_b32 {vr(t0)}, 4, {vr(t0)}")
            for base, src in ((ib, "oimg"), (tb, "otxt")):
                g(f"v_mov_b32 {vr(base + 1)}, %[{src}_hi]")
                g(f"v_add_co_u32 {vr(base)}, vcc, %[{src}_lo], {vr(t0)}")
                g(f"v_addc_co_u32 {vr(base + 1)}, vcc, 0, {vr(base + 1)}, vcc")
        else:
            g(f"v_mad_u64_u32 {vr(addr, 2)}, {sp(S_CMP)}, {vr(left)}, %[ldob], 0")
        g(f"v_sub_u32 {vr(left)}, %[qend], {vr(left)}")
        if not JOINT:
            g(f"v_add_co_u32 {vr(addr)}, vcc, %[obase_lo], {vr(addr)}")
            g(f"v_mov_b32 {vr(ohi)}, %[obase_hi]")
            g(f"v_addc_co_u32 {vr(addr + 1)}, vcc, {vr(ohi)}, {vr(addr + 1)}, vcc")
            g(f"v_and_b32 {vr(t0)}, {lpr - 1}, {lane}")
            g(f"v_lshlrev_b32 {vr(t0)}, 4, {vr(t0)}")
            g(f"v_add_co_u32 {vr(addr)}, vcc, {vr(t0)}, {vr(addr)}")
            g(f"v_addc_co_u32 {vr(addr + 1)}, vcc, 0, {vr(addr + 1)}, vcc")
        g("s_waitcnt lgkmcnt(0)")
        g(f"s_mov_b64 {sp(S_EXEC)}, exec")
        for i in range(32 // rpr):
            if JOINT:
                if i:
                    g(f"s_mov_b64 exec, {sp(S_EXEC)}")
                    g(f"v_add_u32 {vr(j0)}, {rpr}, {vr(j0)}")
                g(f"v_mad_u64_u32 {vr(addr, 2)}, {sp(S_CMP)}, {vr(j0)}, %[ldob], 0")
                g(f"v_cmp_gt_i32 vcc, %[lena], {vr(j0)}")
                g(f"v_cndmask_b32 {vr(EB + 57)}, {vr(tb)}, {vr(ib)}, vcc")
                g(f"v_cndmask_b32 {vr(EB + 58)}, {vr(tb + 1)}, {vr(ib + 1)}, vcc")
                g(f"v_add_co_u32 {vr(addr)}, vcc, {vr(EB + 57)}, {vr(addr)}")
                g(f"v_addc_co_u32 {vr(addr + 1)}, vcc, {vr(EB + 58)}, {vr(addr + 1)}, vcc")
            elif i:
                g(f"s_mov_b64 exec, {sp(S_EXEC)}")
                g(f"v_add_co_u32 {vr(addr)}, vcc, {s_(S_T1)}, {vr(addr)}")
                g(f"v_addc_co_u32 {vr(addr + 1)}, vcc, 0, {vr(addr + 1)}, vcc")
            g(f"v_cmp_lt_i32 vcc, {i * rpr}, {vr(left)}")
            g("s_and_b64 exec, exec, vcc")
            g(f"global_store_dwordx4 {vr(addr, 2)}, {vr(data + 4 * i, 4)}, off nt")  # streamed
        g(f"s_mov_b64 exec, {sp(S_EXEC)}")
        # lse = (m + log2 l) * ln 2 for lanes of the first half-wave, when asked
        skip = g.new_label("nolse")
        g(f"s_cmp_eq_u32 %[has_lse], 0")
        g(f"s_cbranch_scc1 {skip}")
        g(f"v_cmp_gt_i32 vcc, %[qend], {qrow}")
        g("s_and_b64 exec, exec, vcc")
        g(f"v_cmp_gt_u32 vcc, 32, {lane}")
        g("s_and_b64 exec, exec, vcc")
        g(f"s_cbranch_execz {skip}")
        g(f"v_log_f32 {vr(EB + 12)}, {vr(lt)}")
        g("s_nop 0")
        g(f"v_sub_f32 {vr(EB + 12)}, {vr(EB + 12)}, {vr(negm_of(qb))}")
        g(f"v_mul_f32 {vr(EB + 12)}, 0x3f317218, {vr(EB + 12)}")
        g(f"v_cmp_lt_f32 vcc, 0, {vr(lt)}")
        g(f"v_mov_b32 {vr(EB + 14)}, 0xff800000")
        g(f"v_cndmask_b32 {vr(EB + 12)}, {vr(EB + 14)}, {vr(EB + 12)}, vcc")
        g(f"v_lshlrev_b32 {vr(EB + 13)}, 2, {qrow}")
        g(f"global_store_dword {vr(EB + 13)}, {vr(EB + 12)}, %[lsebase]")
        g.label(skip)
        g(f"s_mov_b64 exec, {sp(S_EXEC)}")


def generate():
    g = Gen()
    empty = g.new_label("nokeys")
    prologue(g, empty)
    last_a = g.new_label("lastA")
    last_b = g.new_label("lastB")
    loop = g.new_label("loop")
    fin = g.new_label("fin")
    npass = g.new_label("pass")
    done = g.new_label("done")
    g.label(npass)
    pass_start(g)
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
    g(f"s_cmp_ge_u32 {s_(S_KT)}, {s_(S_NKT1)}")
    g(f"s_cbranch_scc1 {last_b}")
    rb, bb = tile(g, 1)
    g(f"s_cmp_lt_u32 {s_(S_KT)}, {s_(S_NKT1)}")
    g(f"s_cbranch_scc1 {loop}")
    g(f"s_branch {last_a}")
    rescale_block(g, 0, ra, ba)
    rescale_block(g, 1, rb, bb)
    g.label(last_a)
    last_tile(g, 0)
    g(f"s_branch {fin}")
    g.label(last_b)
    last_tile(g, 1)
    g.label(fin)
    epilogue(g)
    # next pass: 256 queries further, loads already issued by the last tile
    g(f"s_sub_u32 {s_(S_NPASS)}, {s_(S_NPASS)}, 1")
    g(f"s_cmp_eq_u32 {s_(S_NPASS)}, 0")
    g(f"s_cbranch_scc1 {done}")
    g(f"s_add_u32 {s_(S_QOFF)}, {s_(S_QOFF)}, {BN * 4}")
    clear_state(g)
    g(f"s_branch {npass}")
    # no keys: every pass stores zero rows
    g.label(empty)
    for i in range(2 * DT * 16):
        g(f"v_accvgpr_write_b32 {ar(O_A + i)}, 0")
    for qb in range(2):
        g(f"v_mov_b32 {vr(LRUN + qb)}, 0")
    epilogue(g)
    g(f"s_sub_u32 {s_(S_NPASS)}, {s_(S_NPASS)}, 1")
    g(f"s_cmp_eq_u32 {s_(S_NPASS)}, 0")
    g(f"s_cbranch_scc1 {done}")
    g(f"s_add_u32 {s_(S_QOFF)}, {s_(S_QOFF)}, {BN * 4}")
    g(f"s_branch {empty}")
    g.label(done)
    return g.lines


def clobbers(hd, pre=False, joint=False):
    configure(hd, pre, joint)
    regs = ([f"v{i}" for i in range(LAST_VGPR + 1)] + [f"a{i}" for i in range(LAST_AGPR + 1)] +
            [f"s{i}" for i in (SGPRS_JOINT if joint else SGPRS)])
    rows = [", ".join(f'"{r}"' for r in regs[i:i + 16]) for i in range(0, len(regs), 16)]
    name = f"{hd}{'j' if joint else 'p' if pre else ''}"
    return (f"// Registers the generated flash_fwd_asm<{hd}, {str(pre).lower()}, {str(joint).lower()}> body owns (gen_attn.py register map).\n"
            f"#define DITK_D{name.upper()}_CLOBBERS \\\n" + "".join(f"  {r}, \\\n" for r in rows) + "\n")


def write_body(path, hd, pre=False, joint=False):
    configure(hd, pre, joint)
    lines = generate()
    with open(path, "w") as f:
        f.write(f"// Generated by gen_attn.py -- the instruction body of flash_fwd_asm<{hd}, {str(pre).lower()}, "
                f"{str(joint).lower()}>.\n")
        for line in lines:
            esc = line.replace("\\", "\\\\").replace('"', '\\"')
            f.write(f'"{esc}\\n"\n')


def main(argv):
    here = os.path.dirname(os.path.abspath(__file__))
    out = os.path.dirname(os.path.abspath(argv[1])) if len(argv) > 1 else here
    for hd, pre, joint in ((128, False, False), (128, True, False), (64, False, False), (64, True, False),
                           (64, True, True)):
        name = f"d{hd}{'j' if joint else 'p' if pre else ''}"
        write_body(os.path.join(out, f"attn_{name}_body.inc"), hd, pre, joint)
        with open(os.path.join(out, f"attn_{name}_clobbers.h"), "w") as f:
            f.write(clobbers(hd, pre, joint))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
