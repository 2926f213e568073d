"""Generate the main loop of the large-tile GEMM (gemm.hip: gemm_kernel_l4) as
gfx950 assembly.

The workgroup computes a 256 (tokens) x 256 (features) tile of
C^T = W A^T with four waves, one per SIMD, each owning a 128 x 128 wave tile:
64 accumulator tiles of v_mfma_f32_16x16x32_bf16 (256 accumulators, all of the
AGPRs).  The compiler cannot hold that working set without copies, so the
registers are placed here:

  AGPR a0..a255    acc[i][j] (4 each): features w_row0 + 16 i + 4 (lane / 16) + e,
                   token a_row0 + 16 j + lane % 16
  VGPR v0..v63     operand set 0: W fragments i (v[4i..4i+3]), then token
                   fragments j (v[32+4j..])
  VGPR v64..v127   operand set 1
  VGPR v128..v139  epilogue temporaries
  SGPR s40..s51    loop state

K advances in 64-k stages through two LDS buffers of 64 KiB (A rows then W
rows, 128 bytes per row -- one L2 line of each operand row per stage -- with
16-byte units XOR-swizzled by row) filled by direct global->LDS DMA.  A stage
is two 32-k chunks of 64 MFMAs; each chunk runs on the operand set read during
the chunk before and reads the next chunk's fragments into the other set (the
even MFMA slots of its first half).  One barrier per stage, between its chunks,
after this wave's DMA of the next stage and its reads of chunk 1 landed: after
it every wave may read the next stage, and this stage's buffer is free, so
chunk 1 issues the DMA of stage min(s + 2, nk - 1) into it (one instruction
every 4 MFMAs).  The first chunk runs peeled, its MFMAs starting from 0.  After
the last stage the accumulators plus bias are rounded to bf16 and staged in LDS
(rows of 272 bytes per wave) for the C++ epilogue.

Every output element accumulates the same MFMAs over the same k order as the
C++ kernels (gemm_kernel), and the bias add and rounding are the same
instructions, so the results are bitwise theirs.

Two wave-tile widths are generated: 128 features (gemm_l4_body.inc, workgroup
tile 256 x 256) and 96 (gemm_l4w96_body.inc, 256 x 192, 192 accumulators) for
the shapes where 192-wide tiles fill the 256 CUs in fewer rounds.

Usage: python gen_gemm.py [dir/any]  (writes gemm_l4_body.inc, gemm_l4w96_body.inc
and gemm_l4_clobbers.h into that directory, default beside this file)
"""
import os
import sys

FJ = 8                  # token fragments per wave tile (128 tokens)


def configure(fi):  # noqa: D401
    """fi feature fragments per wave tile: 8 (wave tile 128 x 128, workgroup tile
    256 x 256) or 6 (128 x 96, workgroup 256 x 192)."""
    global FI, BUF, WOFF, STG_ROW, ND, DMA_SLOTS
    FI = fi
    BUF = (256 + 32 * fi) * 128        # stage buffer: A rows (32 KiB), then W rows
    WOFF = 32 * 1024
    STG_ROW = 32 * fi + 16             # staging row: 16 fi bf16 features + 16 bytes
    ND = 8 + fi                        # DMA instructions per wave and stage (A groups, then W)
    step = fi * FJ // ND                # chunk-1 MFMA slots of the stage's DMAs, evenly spread
    DMA_SLOTS = [step * k + 2 for k in range(ND)]
    assert DMA_SLOTS[-1] < fi * FJ and 2 * (fi + FJ) <= fi * FJ


configure(8)
ROW = 128               # bytes per LDS row (64 k of bf16)

S_A, S_W = 40, 42       # s[40:41], s[42:43] DMA bases of the stage being fetched
S_S, S_NK1, S_SW = 44, 45, 46   # stage index, nk - 1, LDS + 1 KiB wave slice
S_T0, S_T1 = 47, 48
SGPRS = list(range(40, 52))
LAST_VGPR, LAST_AGPR = 139, 255
TMP = 128


def acc(i, j):
    return (i * FJ + j) * 4


def wreg(p, i):
    return p * 64 + i * 4


def xreg(p, j):
    return p * 64 + 32 + j * 4


class Gen:
    def __init__(self):
        self.lines = []
        self.label_n = 0

    def __call__(self, s):
        self.lines.append(s)

    def label(self, name):
        self.lines.append(f"{name}:")

    def new_label(self, stem):
        self.label_n += 1
        return f"L_{stem}_{self.label_n}_%="


def set_dma_bases(g, stage_expr):
    """S_A / S_W = tile bases + min(stage, nk - 1) * 128 bytes."""
    g(f"s_min_u32 s{S_T0}, {stage_expr}, s{S_NK1}")
    g(f"s_lshl_b32 s{S_T0}, s{S_T0}, 7")
    g(f"s_add_u32 s{S_A}, %[a_lo], s{S_T0}")
    g(f"s_addc_u32 s{S_A + 1}, %[a_hi], 0")
    g(f"s_add_u32 s{S_W}, %[w_lo], s{S_T0}")
    g(f"s_addc_u32 s{S_W + 1}, %[w_hi], 0")


def dma_m0(g, k, buf):
    """DMA instruction k (0..7: A groups, 8..15: W groups) of this wave into buffer buf."""
    base = buf * BUF + (WOFF if k >= 8 else 0) + (k % 8) * 4096
    g(f"s_add_u32 m0, s{S_SW}, {base}")


def dma_go(g, k):
    if k < 8:
        g(f"global_load_lds_dwordx4 %[aoff{k}], s[{S_A}:{S_A + 1}]")
    else:
        g(f"global_load_lds_dwordx4 %[woff{k - 8}], s[{S_W}:{S_W + 1}]")


def dma_block(g, buf):
    for k in range(ND):
        dma_m0(g, k, buf)
        g("s_nop 0")
        dma_go(g, k)


def read_frag(g, kind, idx, p, buf, c):
    reg = wreg(p, idx) if kind == "w" else xreg(p, idx)
    base = f"%[rd{kind}{buf}{c}]"
    g(f"ds_read_b128 v[{reg}:{reg + 3}], {base} offset:{idx * 16 * ROW}")


def read_order():
    return [("w", 0), ("x", 0)] + [("w", i) for i in range(1, FI)] + [("x", j) for j in range(1, FJ)]


def chunk(g, p, first, reads, dmas):
    """64 MFMAs on operand set p; reads: (buffer, chunk) of the fragments to read
    into set 1 - p (one per even slot of the first half); dmas: (buffer) the
    stage's DMA goes to, spread over the chunk, or None."""
    order = read_order()
    for m in range(FI * FJ):
        j, i = m // FI, m % FI
        k = DMA_SLOTS.index(m) if dmas is not None and m in DMA_SLOTS else None
        if k is not None:
            dma_m0(g, k, dmas)
        src_c = "0" if first else f"a[{acc(i, j)}:{acc(i, j) + 3}]"
        g(f"v_mfma_f32_16x16x32_bf16 a[{acc(i, j)}:{acc(i, j) + 3}], v[{wreg(p, i)}:{wreg(p, i) + 3}], "
          f"v[{xreg(p, j)}:{xreg(p, j) + 3}], {src_c}")
        if m % 2 == 0 and m // 2 < len(order):
            kind, idx = order[m // 2]
            read_frag(g, kind, idx, 1 - p, *reads)
        if k is not None:
            dma_go(g, k)


def stage(g, buf, first=False, last_check=None):
    """One 64-k stage s (s % 2 == buf): chunk 0 on operand set 0 (read during the
    previous stage) while reading chunk 1 into set 1; the barrier that publishes
    stage s + 1 (this wave's DMA of it landed) and frees buffer s % 2 (every
    wave's reads of it done); chunk 1 on set 1 while reading stage s + 1's chunk 0
    into set 0 and DMAing stage min(s + 2, nk - 1) into buffer s % 2."""
    chunk(g, 0, first, (buf, 1), None)
    g("s_waitcnt vmcnt(0) lgkmcnt(0)")
    g("s_barrier")
    g(f"s_add_u32 s{S_T1}, s{S_S}, 2")
    set_dma_bases(g, f"s{S_T1}")
    chunk(g, 1, False, (1 - buf, 0), buf)
    g(f"s_add_u32 s{S_S}, s{S_S}, 1")
    g("s_waitcnt lgkmcnt(0)")
    if last_check is not None:
        g(f"s_cmp_gt_u32 s{S_S}, s{S_NK1}")
        g(f"s_cbranch_scc1 {last_check}")


def prologue(g):
    # a persistent workgroup's previous tile: every wave's reads of its staged
    # rows are done before the stage DMAs overwrite them
    g("s_waitcnt lgkmcnt(0)")
    g("s_barrier")
    g(f"s_add_u32 s{S_SW}, %[lds], %[wave1k]")
    g(f"s_sub_u32 s{S_NK1}, %[nk], 1")
    g(f"s_mov_b32 s{S_S}, 0")
    # stages 0 and 1 into buffers 0 and 1 (clamped to the last stage)
    for st in range(2):
        g(f"s_mov_b32 s{S_T1}, {st}")
        set_dma_bases(g, f"s{S_T1}")
        dma_block(g, st)
    g(f"s_waitcnt vmcnt({ND})")
    g("s_barrier")
    for kind, idx in read_order():
        read_frag(g, kind, idx, 0, 0, 0)
    g("s_waitcnt lgkmcnt(0)")


def epilogue(g):
    """acc + bias -> bf16 pairs -> this wave's staging rows: token row j*16 + lane%16,
    8-byte unit i*4 + lane/16 (features 4 apart)."""
    g("s_waitcnt vmcnt(0) lgkmcnt(0)")
    g("s_barrier")
    g("s_nop 7")
    g("s_nop 7")
    g("s_nop 7")
    for i in range(FI):
        for j in range(FJ):
            a = acc(i, j)
            for e in range(4):
                g(f"v_accvgpr_read_b32 v{TMP + e}, a{a + e}")
            for e in range(4):
                g(f"v_add_f32 v{TMP + e}, v{TMP + e}, %[b{i * 4 + e}]")
            g(f"v_cvt_pk_bf16_f32 v{TMP + 4}, v{TMP}, v{TMP + 1}")
            g(f"v_cvt_pk_bf16_f32 v{TMP + 5}, v{TMP + 2}, v{TMP + 3}")
            g(f"ds_write_b64 %[stg], v[{TMP + 4}:{TMP + 5}] offset:{j * 16 * STG_ROW + i * 32}")
    g("s_waitcnt lgkmcnt(0)")


def generate():
    g = Gen()
    prologue(g)
    done = g.new_label("done")
    loop = g.new_label("loop")
    # stage 0 peeled (its MFMAs start from 0), then stage pairs (buffers 1, 0)
    stage(g, 0, first=True, last_check=done)
    g.label(loop)
    stage(g, 1, last_check=done)
    stage(g, 0, last_check=done)
    g(f"s_branch {loop}")
    g.label(done)
    epilogue(g)
    return g.lines


def clobbers():
    regs = ([f"v{i}" for i in range(LAST_VGPR + 1)] + [f"a{i}" for i in range(LAST_AGPR + 1)] +
            [f"s{i}" for i in SGPRS])
    rows = [", ".join(f'"{r}"' for r in regs[i:i + 16]) for i in range(0, len(regs), 16)]
    return ("// Registers the generated gemm_kernel_l4 body owns (gen_gemm.py register map).\n"
            "#define DITK_GEMM_L4_CLOBBERS \\\n" + "".join(f"  {r}, \\\n" for r in rows) + "\n")


def write_body(path, fi):
    configure(fi)
    lines = generate()
    with open(path, "w") as f:
        f.write(f"// Generated by gen_gemm.py -- the instruction body of gemm_kernel_l4<FI = {fi}>.\n")
        for line in lines:
            esc = line.replace("\\", "\\\\").replace('"', '\\"')
            f.write(f'"{esc}\\n"\n')


def main(argv):
    here = os.path.dirname(os.path.abspath(__file__))
    out = os.path.dirname(os.path.abspath(argv[1])) if len(argv) > 1 else here
    write_body(os.path.join(out, "gemm_l4_body.inc"), 8)
    write_body(os.path.join(out, "gemm_l4w96_body.inc"), 6)
    configure(8)
    with open(os.path.join(out, "gemm_l4_clobbers.h"), "w") as f:
        f.write(clobbers())
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
