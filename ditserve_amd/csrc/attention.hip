// Varlen block-diagonal flash attention (forward, non-causal), bf16 MFMA.
//
// Packed layout: Q [Tq, ldq], K [Tk, ldk] with head h at columns [h*HD, h*HD+HD);
// segment m's queries [cu_q[m], cu_q[m+1]) attend only to keys
// [cu_k[m], cu_k[m+1]).  Self-attention (cu_q == cu_k), text cross-attention
// (cu_k = 512-row text blocks) and SD3.5 joint attention (image+text joint
// segments) are all this one kernel.
//
// V is consumed transposed: Vt [heads][HD][Tpad], where segment m's keys start
// at the 64-aligned column pk[m] = 64 * sum_{m'<m} ceil(len_k[m'] / 64) and the
// padding columns are zero.  ditk_transpose_v produces it.
//
// A workgroup is four waves of 64 queries of one (segment, head), one wave per
// SIMD; K/Vt tiles of 64 keys are staged through LDS by direct global->LDS DMA.
// Each wave computes
//   S^T = K Q^T        (A = K rows from LDS, B = Q held in AGPRs)
//   P^T = exp2(S^T * scale*log2e - m)   (online softmax, fp32)
//   O^T += Vt P^T      (A = Vt rows from LDS, B = P^T straight from registers)
// with v_mfma_f32_32x32x16_bf16.  The K rows fed to the first MFMA are permuted
// (kperm) so that the S^T accumulator registers of each lane are exactly the
// B-operand layout of the second MFMA: no shuffles between the two products.
// Each lane owns one query of each 32-query block, so softmax statistics are
// per-lane scalars combined across the two half-waves with one exchange.  The
// running max is raised lazily: a tile is redone against its own max only when a
// lane's row sum over its 64 keys exceeds 2^8.  The loop body is generated
// assembly (gen_attn.py), its registers placed by hand.
//
// Query tiles start at each segment's first query and the key loop starts at
// each segment's first key, so results are independent of packing: a request
// packed with others is bitwise equal to the same request run alone.
//
// PRE: Q arrives multiplied by softmax_scale*log2(e) — the producer folds that
// factor into its QK-norm weight, so Q is still rounded to bf16 once.  The S^T
// accumulators then start from a register block holding -m instead of zero,
// and P = exp2(S) takes no fma: every live S register holds q.k - m_run, and
// whenever m_run moves by d the live S registers and the block move by -d.
//
// JOINT (with PRE, head_dim 64): each joint segment's rows come from two packed
// sources — row j of segment m is row cu_a[m] + j of the "a" operand (image
// tokens) while j < len_a(m), else row cu_b[m] + j - len_a(m) of the "b"
// operand (text tokens) — for Q, K and O alike, so SD3.5's image and text
// projections feed joint attention, and take its output, without a gather or
// scatter copy.  Results are bitwise those of the gathered layout.
#include <mutex>

#include "ditk_common.h"
#include "attn_d128_clobbers.h"
#include "attn_d128p_clobbers.h"
#include "attn_d64_clobbers.h"
#include "attn_d64p_clobbers.h"
#include "attn_d64j_clobbers.h"

namespace {

constexpr int BN = 64;        // keys per tile

// S^T row m of a 32-key MFMA tile holds key kperm(m): with the D layout
// row = (v/4)*8 + (lane/32)*4 + v%4, this puts key (v/8)*16 + (lane/32)*8 + v%8
// in accumulator register v — the B-operand k-slot order of the PV product.
__device__ __forceinline__ int kperm(int m) {
  return ((m >> 4) << 4) | (((m >> 2) & 1) << 3) | (((m >> 3) & 1) << 2) | (m & 3);
}


// segment m and tile index within it for the t-th (0-based) tile of `tile`-sized
// tiles laid over the segments of cu; returns -1 if t is past the last tile.
__device__ __forceinline__ int locate_tile(const int32_t* __restrict__ cu, int nseg, int tile, int& t) {
  int prev = cu[0];
  for (int m = 0; m < nseg; ++m) {
    int next = cu[m + 1];
    int n = (next - prev + tile - 1) / tile;
    if (t < n) return m;
    t -= n;
    prev = next;
  }
  return -1;
}

// 64-aligned start column of segment m in the transposed V layout
__device__ __forceinline__ int padded_key_start(const int32_t* __restrict__ cu, int m) {
  int pk = 0;
  for (int i = 0; i < m; ++i) pk += ((cu[i + 1] - cu[i] + BN - 1) / BN) * BN;
  return pk;
}

// LDS tile layouts: rows of 16-byte chunks, grouped 8 chunks (128 B) per row
// per group, and XOR-swizzled inside the group by the row:
//   slot(row, u) = (u / 8) * rows * 8 + row * 8 + ((u % 8) ^ ((row >> 1) & 7))
//   K stage : rows = BN keys, u = head-dim chunk (8 dims each), HD/64 groups
//   Vt stage: rows = HD dims, u = key chunk (8 keys each), 1 group
// A DMA instruction fills 64 consecutive slots = 8 rows x 128 contiguous bytes;
// 16 consecutive lanes reading one chunk of 16 different rows hit 16 distinct
// 16-byte bank groups; each lane's read address is one of 4 per-lane bases
// plus a compile-time offset.
// head_dim 128 or 64, 64 queries per wave (two 32-query blocks), one wave per
// SIMD: four waves and 256 queries per workgroup.  The C++ side locates the work
// item and computes per-lane addresses; the body is generated assembly
// (gen_attn.py -> attn_d{128,64}[p|j]_body.inc) with its registers
// placed by hand: O^T and Q in AGPRs, S^T and P in VGPRs, so that the whole
// working set stays in registers.
#define DITK_ATTN_ASM_OPERANDS                                                                                      \
  [qbase_lo] "s"(su((uint32_t)qbase)), [qbase_hi] "s"(su((uint32_t)(qbase >> 32))), [kdma_lo] "s"(su((uint32_t)kdma)), \
      [kdma_hi] "s"(su((uint32_t)(kdma >> 32))), [vdma_lo] "s"(su((uint32_t)vdma)),                               \
      [vdma_hi] "s"(su((uint32_t)(vdma >> 32))), [lds_k] "s"(su(lds_k)), [lds_v] "s"(su(lds_v)),                   \
      [nkt] "s"(su(nkt)), [valid_last] "s"(su(valid_last)), [ktile] "s"(su(ktile)), [wave1k] "s"(su(wave1k)),      \
      [lds_o] "s"(su(lds_o)), [npass] "s"(su(npass)), [ldqb] "s"(su(ldqb)), [sc] "s"(sc), [qend] "s"(su(q_end)), [ldob] "s"(su(ldob)), [obase_lo] "s"(su((uint32_t)obase)),             \
      [obase_hi] "s"(su((uint32_t)(obase >> 32))), [has_lse] "s"(su(has_lse)), [lsebase] "s"(su64(lsebase)),      \
      [kaddr0] "v"(kaddr[0]), [kaddr1] "v"(kaddr[1]), [kaddr2] "v"(kaddr[2]), [kaddr3] "v"(kaddr[3]),             \
      [vaddr0] "v"(vaddr[0]), [vaddr1] "v"(vaddr[1]), [vaddr2] "v"(vaddr[2]), [vaddr3] "v"(vaddr[3]),             \
      [koff0] "v"(koff[0]), [koff1] "v"(koff[1]), [koff2] "v"(koff[2]), [koff3] "v"(koff[3]),                     \
      [koffl0] "v"(koffl[0]), [koffl1] "v"(koffl[1]), [koffl2] "v"(koffl[2]), [koffl3] "v"(koffl[3]),             \
      [voff0] "v"(voff[0]), [voff1] "v"(voff[1]), [voff2] "v"(voff[2]), [voff3] "v"(voff[3]),                     \
      [lane] "v"(lanev), [qrow0] "v"(qrow0), [qrow1] "v"(qrow1)
// Pre-scaled q: the body's -m blocks take 32 more VGPRs, so the per-lane values
// it reads only outside the key loop arrive in AGPRs
#define DITK_ATTN_ASM_OPERANDS_PRE                                                                                  \
  [qbase_lo] "s"(su((uint32_t)qbase)), [qbase_hi] "s"(su((uint32_t)(qbase >> 32))), [kdma_lo] "s"(su((uint32_t)kdma)), \
      [kdma_hi] "s"(su((uint32_t)(kdma >> 32))), [vdma_lo] "s"(su((uint32_t)vdma)),                               \
      [vdma_hi] "s"(su((uint32_t)(vdma >> 32))), [lds_k] "s"(su(lds_k)), [lds_v] "s"(su(lds_v)),                   \
      [nkt] "s"(su(nkt)), [valid_last] "s"(su(valid_last)), [ktile] "s"(su(ktile)), [wave1k] "s"(su(wave1k)),      \
      [lds_o] "s"(su(lds_o)), [npass] "s"(su(npass)), [ldqb] "s"(su(ldqb)), [qend] "s"(su(q_end)), [ldob] "s"(su(ldob)), [obase_lo] "s"(su((uint32_t)obase)),                           \
      [obase_hi] "s"(su((uint32_t)(obase >> 32))), [has_lse] "s"(su(has_lse)), [lsebase] "s"(su64(lsebase)),      \
      [kaddr0] "v"(kaddr[0]), [kaddr1] "v"(kaddr[1]), [kaddr2] "v"(kaddr[2]), [kaddr3] "v"(kaddr[3]),             \
      [vaddr0] "v"(vaddr[0]), [vaddr1] "v"(vaddr[1]), [vaddr2] "v"(vaddr[2]), [vaddr3] "v"(vaddr[3]),             \
      [koff0] "a"(koff[0]), [koff1] "a"(koff[1]), [koff2] "a"(koff[2]), [koff3] "a"(koff[3]),                     \
      [koffl0] "a"(koffl[0]), [koffl1] "a"(koffl[1]), [koffl2] "a"(koffl[2]), [koffl3] "a"(koffl[3]),             \
      [voff0] "v"(voff[0]), [voff1] "v"(voff[1]), [voff2] "v"(voff[2]), [voff3] "v"(voff[3]),                     \
      [lane] "a"(lanev), [qrow0] "a"(qrow0), [qrow1] "a"(qrow1)
// Joint sources (with pre-scaled q): the two K and O source bases of the segment
// (the text ones shifted back by len_img rows), len_img, the segment's first
// joint row, per-lane Q row addresses and the K rows of each DMA instruction
#define DITK_ATTN_ASM_OPERANDS_JOINT                                                                                \
  DITK_ATTN_ASM_OPERANDS_PRE, [ktxt_lo] "s"(su((uint32_t)ktxt)), [ktxt_hi] "s"(su((uint32_t)(ktxt >> 32))),        \
      [lena] "s"(su(len_a)), [qseg] "s"(su(qseg)), [oimg_lo] "s"(su((uint32_t)oimg)),                              \
      [oimg_hi] "s"(su((uint32_t)(oimg >> 32))), [otxt_lo] "s"(su((uint32_t)otxt)),                                \
      [otxt_hi] "s"(su((uint32_t)(otxt >> 32))), [qa0lo] "a"((uint32_t)qa[0]), [qa0hi] "a"((uint32_t)(qa[0] >> 32)), \
      [qa1lo] "a"((uint32_t)qa[1]), [qa1hi] "a"((uint32_t)(qa[1] >> 32)), [krow0] "a"(krow_of[0]),                  \
      [krow1] "a"(krow_of[1]), [krow2] "a"(krow_of[2]), [krow3] "a"(krow_of[3])
constexpr int kXcdChunk = 32;  // work items per XCD chunk (one per CU of an XCD)
template <int HD, bool PRE, bool JOINT = false>
__global__ __launch_bounds__(256, 1) void flash_fwd_asm(
    const bf16_t* __restrict__ Q, int64_t ldq, const bf16_t* __restrict__ Kp, int64_t ldk,
    const bf16_t* __restrict__ Vt, int64_t vt_ld, int64_t vt_hs, bf16_t* __restrict__ O, int64_t ldo,
    float* __restrict__ lse, int64_t lse_ld, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ cu_k, int nseg, int heads, int np, float scale_log2,
    const bf16_t* __restrict__ Qb = nullptr, const bf16_t* __restrict__ Kb = nullptr, bf16_t* __restrict__ Ob = nullptr,
    const int32_t* __restrict__ cu_a = nullptr, const int32_t* __restrict__ cu_b = nullptr) {
  static_assert(!JOINT || (PRE && HD == 64), "joint sources: pre-scaled head_dim 64");
  constexpr int NW = 4, BM = 256;
  constexpr int ND = HD / 32;  // DMA instructions per wave and operand per tile
  __shared__ u32x4_t Ks[2][BN * HD / 8];
  __shared__ u32x4_t Vs[2][HD * 8];
  constexpr int OPITCH = HD * 2 + 8;  // output staging row pitch (bytes), 32 rows per wave
  __shared__ u32x4_t Os[4 * 32 * OPITCH / 16];
  // A work item is np consecutive 256-query tiles of one (segment, head), run as
  // passes of the body (the next pass's loads issued under the current pass's
  // last key tile).  Items in segment-major order (segment, then head, then
  // tile), dealt to the 8 XCDs (workgroup b runs on XCD b % 8) in chunks of
  // kXcdChunk consecutive items: every XCD gets every 8th chunk, so a ragged
  // batch spreads evenly over the XCDs, and the items running on one XCD at a
  // time are tiles of the same (segment, head), sharing its K and Vt in that
  // XCD's L2.  The grid is a multiple of 8 chunks; items past the last exit.
  const int b = blockIdx.x;
  const int j = b >> 3;
  int t = ((j / kXcdChunk) * 8 + (b & 7)) * kXcdChunk + j % kXcdChunk;
  int seg = -1, head = 0, npass = 0;
  for (int m = 0, prev = cu_q[0]; m < nseg; ++m) {
    const int next = cu_q[m + 1];
    const int ntile = (next - prev + BM - 1) / BM;
    const int n = (ntile + np - 1) / np;
    if (t < n * heads) {
      seg = m;
      head = t / n;
      t = (t - head * n) * np;
      npass = min(np, ntile - t);
      break;
    }
    t -= n * heads;
    prev = next;
  }
  if (seg < 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int q_end = cu_q[seg + 1];
  const int qrow0 = cu_q[seg] + t * BM + wave * 64 + l32;
  const int qrow1 = qrow0 + 32;
  const int k_beg = cu_k[seg], k_len = max(cu_k[seg + 1] - k_beg, 0);
  // nkt == 0 (no keys): the body stores zero rows and lse = -inf, issuing no DMA
  const int nkt = (k_len + BN - 1) / BN;
  const int valid_last = k_len - (nkt - 1) * BN;
  const int pk = padded_key_start(cu_k, seg);
  // Q rows past the segment end read its last row (their outputs are not stored);
  // the body forms each lane's 64-bit row address from qbase, its row and ldq
  const uint64_t qbase = (uint64_t)(uintptr_t)(Q + (int64_t)head * HD);
  uint64_t kdma = (uint64_t)(uintptr_t)(Kp + (int64_t)head * HD + (int64_t)k_beg * ldk);
  // joint: row j of the segment is row a0 + j of the "a" (image) operands while
  // j < len_a, else row b0 + j - len_a of the "b" (text) operands
  int len_a = 0, qseg = 0;
  uint64_t ktxt = 0, oimg = 0, otxt = 0, qa[2] = {0, 0};
  uint32_t krow_of[4] = {};
  if constexpr (JOINT) {
    const int a0 = cu_a[seg], b0 = cu_b[seg];
    len_a = cu_a[seg + 1] - a0;
    qseg = cu_q[seg];
    kdma = (uint64_t)(uintptr_t)(Kp + (int64_t)head * HD + (int64_t)a0 * ldk);
    ktxt = (uint64_t)(uintptr_t)(Kb + (int64_t)head * HD) + (uint64_t)((int64_t)(b0 - len_a) * ldk * 2);
    oimg = (uint64_t)(uintptr_t)(O + (int64_t)head * HD + (int64_t)a0 * ldo);
    otxt = (uint64_t)(uintptr_t)(Ob + (int64_t)head * HD) + (uint64_t)((int64_t)(b0 - len_a) * ldo * 2);
    for (int qb = 0; qb < 2; ++qb) {
      const int jq = min(qb ? qrow1 : qrow0, q_end - 1) - qseg;
      const bf16_t* src = jq < len_a ? Q + (int64_t)(a0 + jq) * ldq : Qb + (int64_t)(b0 + jq - len_a) * ldq;
      qa[qb] = (uint64_t)(uintptr_t)(src + (int64_t)head * HD + hh * 8);
    }
  }
  const uint64_t vdma = (uint64_t)(uintptr_t)(Vt + (int64_t)head * vt_hs + pk);
  const uint32_t ktile = (uint32_t)(BN * ldk * 2);
  const uint32_t ldkb = (uint32_t)(ldk * 2);
  // LDS read bases (bytes within a stage): K rows permuted by kperm, 16-byte
  // chunks swizzled by the row (the LDS tile layout above)
  const int kr = kperm(l32), kg = (kr >> 1) & 7, vg = (l32 >> 1) & 7;
  // LDS read addresses (stage 0; the other stage is an immediate offset), K DMA
  // source offsets (koffl: the last tile's, rows past the segment end reading its
  // last row) and Vt DMA source offsets, per lane
  const uint32_t lds_k = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4_t*)&Ks[0][0];
  const uint32_t lds_v = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4_t*)&Vs[0][0];
  const uint32_t lds_o = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4_t*)&Os[0] +
                         (uint32_t)wave_u * (32 * OPITCH);
  uint32_t kaddr[4], vaddr[4], koff[4] = {}, koffl[4] = {}, voff[4] = {};
  const int lrow = lane >> 3;
  const int lsw0 = ((lane & 7) ^ ((lane >> 4) & 7)) * 8;
  const int lsw1 = ((lane & 7) ^ (((lane >> 4) + 4) & 7)) * 8;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kaddr[i] = lds_k + (uint32_t)(kr * 8 + ((i * 2 + hh) ^ kg)) * 16;
    vaddr[i] = lds_v + (uint32_t)(l32 * 8 + ((i * 2 + hh) ^ vg)) * 16;
  }
#pragma unroll
  for (int i = 0; i < ND; ++i) {
    const int g = i * NW + wave_u;
    const int grp = g / (BN / 8), r8 = g % (BN / 8);
    const uint32_t krow = (uint32_t)(r8 * 8 + lrow);
    const uint32_t kcolb = (uint32_t)(grp * 64 + ((r8 & 1) ? lsw1 : lsw0)) * 2;
    koff[i] = krow * ldkb + kcolb;
    koffl[i] = min(krow, (uint32_t)(valid_last - 1)) * ldkb + kcolb;
    if constexpr (JOINT) krow_of[i] = krow;
    voff[i] = (uint32_t)((int64_t)(g * 8 + lrow) * vt_ld + ((g & 1) ? lsw1 : lsw0)) * 2;
  }
  const uint32_t wave1k = (uint32_t)wave_u * 1024u;
  const uint32_t lanev = (uint32_t)lane;
  const uint64_t obase = (uint64_t)(uintptr_t)(O + (int64_t)head * HD);
  const uint32_t ldob = (uint32_t)(ldo * 2);
  const uint32_t ldqb = (uint32_t)(ldq * 2);
  const uint64_t lsebase = (uint64_t)(uintptr_t)(lse != nullptr ? lse + (int64_t)head * lse_ld : lse);
  const uint32_t has_lse = lse != nullptr;
  // scalar operands: wave-uniform values, made SGPR-resident explicitly
  auto su = [](uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); };
  auto su64 = [&](uint64_t x) { return ((uint64_t)su((uint32_t)(x >> 32)) << 32) | su((uint32_t)x); };
  const float sc = __builtin_bit_cast(float, su(__builtin_bit_cast(uint32_t, scale_log2)));
  if constexpr (HD == 128 && !PRE) {
    asm volatile(
#include "attn_d128_body.inc"
        : : DITK_ATTN_ASM_OPERANDS : DITK_D128_CLOBBERS "vcc", "scc", "memory");
  } else if constexpr (HD == 64 && !PRE) {
    asm volatile(
#include "attn_d64_body.inc"
        : : DITK_ATTN_ASM_OPERANDS : DITK_D64_CLOBBERS "vcc", "scc", "memory");
  } else if constexpr (JOINT) {
    (void)sc;
    asm volatile(
#include "attn_d64j_body.inc"
        : : DITK_ATTN_ASM_OPERANDS_JOINT : DITK_D64J_CLOBBERS "vcc", "scc", "memory");
  } else if constexpr (HD == 128) {
    (void)sc;
    asm volatile(
#include "attn_d128p_body.inc"
        : : DITK_ATTN_ASM_OPERANDS_PRE : DITK_D128P_CLOBBERS "vcc", "scc", "memory");
  } else {
    (void)sc;
    asm volatile(
#include "attn_d64p_body.inc"
        : : DITK_ATTN_ASM_OPERANDS_PRE : DITK_D64P_CLOBBERS "vcc", "scc", "memory");
  }
}

// V [Tk, ldv] (head h at columns h*HD..) -> Vt [heads][HD][vt_ld], per-segment
// 64-aligned columns, zero padding.  One workgroup per (64-key tile, head).
// With cu_a != nullptr the segment's rows come from V (rows cu_a[m] + j) and Vb
// (rows cu_b[m] + j - len_a(m)), as in the joint attention kernel.
template <int HD>
__global__ __launch_bounds__(256) void transpose_v_kernel(const bf16_t* __restrict__ V, int64_t ldv,
                                                          bf16_t* __restrict__ Vt, int64_t vt_ld,
                                                          int64_t vt_hs, const int32_t* __restrict__ cu,
                                                          int nseg, const bf16_t* __restrict__ Vb,
                                                          const int32_t* __restrict__ cu_a,
                                                          const int32_t* __restrict__ cu_b) {
  // LDS tile of 32-bit words: word (d, p) holds keys 2p (low half) and 2p + 1 of
  // head dim d, so a 16-byte read gives 8 consecutive keys of one d.  Row pitch 36
  // words (16-byte aligned rows); key-pair groups of 4 rotated by d / 8 so the
  // writes of one wave (16 d-chunks x 4 key pairs) fall two lanes per bank.
  constexpr int PW = 36;
  __shared__ uint32_t tile[HD * PW];
  auto col = [](int d, int p) { return (p + 4 * ((d >> 3) & 7)) & 31; };
  int t = blockIdx.x;
  const int head = blockIdx.y;
  const int seg = locate_tile(cu, nseg, BN, t);
  if (seg < 0) return;
  const int k0 = cu[seg] + t * BN;
  const int k_end = cu[seg + 1];
  const int col0 = padded_key_start(cu, seg) + t * BN;
  const bf16_t* Vh = V + (int64_t)head * HD;
  constexpr int CH = HD / 8;
  // row r of this tile (zero past the segment end)
  auto load_row = [&](int r, int ch) {
    u32x4_t v = u32x4_t{0, 0, 0, 0};
    if (k0 + r < k_end) {
      if (cu_a != nullptr) {
        const int j = t * BN + r, len_a = cu_a[seg + 1] - cu_a[seg];
        const bf16_t* src = j < len_a ? Vh + (int64_t)(cu_a[seg] + j) * ldv
                                      : Vb + (int64_t)head * HD + (int64_t)(cu_b[seg] + j - len_a) * ldv;
        v = *reinterpret_cast<const u32x4_t*>(src + ch * 8);
      } else {
        v = *reinterpret_cast<const u32x4_t*>(Vh + (int64_t)(k0 + r) * ldv + ch * 8);
      }
    }
    return v;
  };
  // 16-byte chunk ch of rows 2p and 2p + 1 (a wave reads CH chunks of 64 / CH rows pairs)
  for (int idx = threadIdx.x; idx < (BN / 2) * CH; idx += 256) {
    const int ch = idx % CH, p = idx / CH;
    const u32x4_t lo = load_row(2 * p, ch), hi = load_row(2 * p + 1, ch);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = ch * 8 + 2 * i;
      tile[d * PW + col(d, p)] = (lo[i] & 0xffffu) | (hi[i] << 16);
      tile[(d + 1) * PW + col(d + 1, p)] = (lo[i] >> 16) | (hi[i] & 0xffff0000u);
    }
  }
  __syncthreads();
  bf16_t* out = Vt + (int64_t)head * vt_hs + col0;
  for (int idx = threadIdx.x; idx < HD * (BN / 8); idx += 256) {
    const int d = idx >> 3, kc = idx & 7;  // keys 8 kc .. 8 kc + 7 = key pairs 4 kc .. 4 kc + 3
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(&tile[d * PW + col(d, 4 * kc)]);
    *reinterpret_cast<u32x4_t*>(out + (int64_t)d * vt_ld + kc * 8) = w;
  }
}

}  // namespace

// Columns of the transposed-V buffer needed for Tk keys in nseg segments (upper bound).
DITK_EXPORT int64_t ditk_vt_columns(int64_t Tk, int nseg) {
  return ((Tk + BN - 1) / BN + (int64_t)nseg) * BN;
}

namespace {
int transpose_launch(const void* v, const void* vb, int64_t ldv, void* vt, int64_t vt_ld, int Tk, int heads,
                     int head_dim, const int32_t* cu_k, const int32_t* cu_a, const int32_t* cu_b, int nseg,
                     hipStream_t stream) {
  DITK_REQUIRE(cu_k && (Tk == 0 || (v && vt)), "ditk_transpose_v: null tensor");
  DITK_REQUIRE(head_dim == 64 || head_dim == 128, "ditk_transpose_v: head_dim must be 64 or 128");
  DITK_REQUIRE(nseg > 0 && heads > 0 && Tk >= 0, "ditk_transpose_v: bad sizes");
  DITK_REQUIRE(ldv % 8 == 0 && vt_ld % 8 == 0, "ditk_transpose_v: leading dims must be multiples of 8");
  DITK_REQUIRE(vt_ld >= ditk_vt_columns(Tk, nseg), "ditk_transpose_v: vt_ld=%lld < required %lld",
               (long long)vt_ld, (long long)ditk_vt_columns(Tk, nseg));
  DITK_REQUIRE(((uintptr_t)v % 16) == 0 && ((uintptr_t)vt % 16) == 0 && ((uintptr_t)vb % 16) == 0,
               "ditk_transpose_v: misaligned");
  if (Tk == 0) return 0;
  dim3 grid((unsigned)((Tk + BN - 1) / BN + nseg), (unsigned)heads);
  const int64_t hs = (int64_t)head_dim * vt_ld;
  if (head_dim == 128)
    transpose_v_kernel<128><<<grid, 256, 0, stream>>>((const bf16_t*)v, ldv, (bf16_t*)vt, vt_ld, hs, cu_k, nseg,
                                                       (const bf16_t*)vb, cu_a, cu_b);
  else
    transpose_v_kernel<64><<<grid, 256, 0, stream>>>((const bf16_t*)v, ldv, (bf16_t*)vt, vt_ld, hs, cu_k, nseg,
                                                      (const bf16_t*)vb, cu_a, cu_b);
  return ditk_check_launch("ditk_transpose_v");
}
}  // namespace

DITK_EXPORT int ditk_transpose_v(const void* v, int64_t ldv, void* vt, int64_t vt_ld, int Tk,
                                 int heads, int head_dim, const int32_t* cu_k, int nseg,
                                 hipStream_t stream) {
  return transpose_launch(v, nullptr, ldv, vt, vt_ld, Tk, heads, head_dim, cu_k, nullptr, nullptr, nseg, stream);
}

DITK_EXPORT int ditk_transpose_v_joint(const void* v_a, const void* v_b, int64_t ldv, void* vt, int64_t vt_ld,
                                       int T_joint, int heads, int head_dim, const int32_t* cu_a,
                                       const int32_t* cu_b, const int32_t* cu_joint, int nseg, hipStream_t stream) {
  DITK_REQUIRE(v_a && v_b && cu_a && cu_b, "ditk_transpose_v_joint: null tensor");
  return transpose_launch(v_a, v_b, ldv, vt, vt_ld, T_joint, heads, head_dim, cu_joint, cu_a, cu_b, nseg, stream);
}

namespace {
// shared checks and launch of both attention entry points; sl2 = the factor that
// takes q.k to log2 units inside the kernel (unused when pre)
int flash_launch(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* vt, int64_t vt_ld, void* o,
                 int64_t ldo, float* lse, int64_t lse_ld, const int32_t* cu_q, const int32_t* cu_k, int nseg, int Tq,
                 int heads, int head_dim, float sl2, bool pre, hipStream_t stream, const void* qb = nullptr,
                 const void* kb = nullptr, void* ob = nullptr, const int32_t* cu_a = nullptr,
                 const int32_t* cu_b = nullptr) {
  const bool joint = cu_a != nullptr;
  DITK_REQUIRE(!joint || (pre && qb && kb && ob && cu_b), "ditk_joint_attn: needs both sources and both tables");
  DITK_REQUIRE(!joint || (((uintptr_t)qb % 16) == 0 && ((uintptr_t)kb % 16) == 0 && ((uintptr_t)ob % 8) == 0),
               "ditk_joint_attn: misaligned tensor");
  // q and o may be NULL when there are no queries (empty tensors)
  DITK_REQUIRE(k && vt && cu_q && cu_k && (Tq == 0 || (q && o)), "ditk_flash_attn_varlen: null tensor");
  DITK_REQUIRE(head_dim == 64 || head_dim == 128, "ditk_flash_attn_varlen: head_dim must be 64 or 128, got %d", head_dim);
  DITK_REQUIRE(nseg > 0 && heads > 0 && Tq >= 0, "ditk_flash_attn_varlen: bad sizes");
  DITK_REQUIRE(ldq % 8 == 0 && ldk % 8 == 0 && ldo % 4 == 0 && vt_ld % 8 == 0,
               "ditk_flash_attn_varlen: leading dims must be multiples of 8 (ldo of 4)");
  DITK_REQUIRE(((uintptr_t)q % 16) == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)vt % 16) == 0 &&
               ((uintptr_t)o % 8) == 0, "ditk_flash_attn_varlen: misaligned tensor");
  // the kernel addresses a 64-row K tile and an HD-row Vt tile with 32-bit element offsets
  DITK_REQUIRE(ldk < (1ll << 24) && vt_ld < (1ll << 24), "ditk_flash_attn_varlen: ldk / vt_ld too large");
  if (Tq == 0) return 0;
  const int64_t hs = (int64_t)head_dim * vt_ld;
  // Q and O rows are addressed in 64 bits; the lse rows and tile offsets in 32
  DITK_REQUIRE(Tq < (1 << 30) && ldk < (1ll << 23) && vt_ld < (1ll << 23),
               "ditk_flash_attn_varlen: tensor too large for 32-bit lane offsets");
  // passes per work item: several query tiles per workgroup when the segments
  // have few keys (vt_ld / nseg bounds the mean key count from above), so the
  // next tile's loads hide under the current one's last key tile, as long as
  // the items still fill the CUs at least twice over (512 items at 4 tiles each)
  const int np = (!joint && vt_ld / nseg <= 2048 && (int64_t)((Tq + 255) / 256) * heads >= 2048) ? 4 : 1;
  const int tiles_bound = ((Tq + 255) / 256 + nseg + np - 1) / np + nseg;
  int64_t nblocks = (int64_t)tiles_bound * heads;
  nblocks = (nblocks + 8 * kXcdChunk - 1) / (8 * kXcdChunk) * (8 * kXcdChunk);
  DITK_REQUIRE(nblocks < (1ll << 31), "ditk_flash_attn_varlen: grid too large");
  auto kern = joint ? flash_fwd_asm<64, true, true>
              : head_dim == 128 ? (pre ? flash_fwd_asm<128, true> : flash_fwd_asm<128, false>)
                                : (pre ? flash_fwd_asm<64, true> : flash_fwd_asm<64, false>);
  kern<<<(unsigned)nblocks, 256, 0, stream>>>((const bf16_t*)q, ldq, (const bf16_t*)k, ldk, (const bf16_t*)vt, vt_ld,
                                              hs, (bf16_t*)o, ldo, lse, lse_ld, cu_q, cu_k, nseg, heads, np, sl2,
                                              (const bf16_t*)qb, (const bf16_t*)kb, (bf16_t*)ob, cu_a, cu_b);
  return ditk_check_launch("ditk_flash_attn_varlen");
}
}  // namespace

DITK_EXPORT int ditk_flash_attn_varlen(const void* q, int64_t ldq, const void* k, int64_t ldk,
                                       const void* vt, int64_t vt_ld, void* o, int64_t ldo,
                                       float* lse, int64_t lse_ld, const int32_t* cu_q,
                                       const int32_t* cu_k, int nseg, int Tq, int heads,
                                       int head_dim, float softmax_scale, hipStream_t stream) {
  DITK_REQUIRE(softmax_scale > 0.f, "ditk_flash_attn_varlen: softmax_scale must be > 0");
  return flash_launch(q, ldq, k, ldk, vt, vt_ld, o, ldo, lse, lse_ld, cu_q, cu_k, nseg, Tq, heads, head_dim,
                      softmax_scale * 1.4426950408889634f, false, stream);
}

DITK_EXPORT int ditk_flash_attn_varlen_q_prescaled(const void* q, int64_t ldq, const void* k, int64_t ldk,
                                                   const void* vt, int64_t vt_ld, void* o, int64_t ldo,
                                                   float* lse, int64_t lse_ld, const int32_t* cu_q,
                                                   const int32_t* cu_k, int nseg, int Tq, int heads,
                                                   int head_dim, hipStream_t stream) {
  return flash_launch(q, ldq, k, ldk, vt, vt_ld, o, ldo, lse, lse_ld, cu_q, cu_k, nseg, Tq, heads, head_dim,
                      1.0f, true, stream);
}

DITK_EXPORT int ditk_joint_attn_q_prescaled(const void* q_a, const void* q_b, int64_t ldq, const void* k_a,
                                            const void* k_b, int64_t ldk, const void* vt, int64_t vt_ld, void* o_a,
                                            void* o_b, int64_t ldo, const int32_t* cu_a, const int32_t* cu_b,
                                            const int32_t* cu_joint, int nseg, int T_joint, int heads,
                                            int head_dim, hipStream_t stream) {
  DITK_REQUIRE(head_dim == 64, "ditk_joint_attn_q_prescaled: head_dim must be 64, got %d", head_dim);
  DITK_REQUIRE(cu_a && cu_b, "ditk_joint_attn_q_prescaled: null segment table");
  return flash_launch(q_a, ldq, k_a, ldk, vt, vt_ld, o_a, ldo, nullptr, 0, cu_joint, cu_joint, nseg, T_joint, heads,
                      head_dim, 1.0f, true, stream, q_b, k_b, o_b, cu_a, cu_b);
}

// ---------------------------------------------------------------------------
// Allocation-free attention: the transposed-V staging lives in a file-scope
// device array instead of a caller- or library-allocated buffer.  Each GPU holds
// its own copy of the array (kScratchBytes) until the process ends; its device
// address is looked up once per device, with that device current, and only that
// address is handed to kernels.  Every call on a GPU shares the array, so calls
// that overlap on one GPU (different streams) race.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kScratchBytes = size_t(64) << 20;  // DITK_NOALLOC_SCRATCH_BYTES of include/ditk.h
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

// device address of `scratch` on the current device (nullptr + message on failure)
void* scratch_ptr() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    ditk_set_error("ditk_flash_attn_varlen_noalloc: no usable current device (%s)", hipGetErrorString(e));
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      ditk_set_error("ditk_flash_attn_varlen_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

DITK_EXPORT int ditk_flash_attn_varlen_noalloc(const void* q, int64_t ldq, const void* k, int64_t ldk,
                                               const void* v, int64_t ldv, void* o, int64_t ldo, float* lse,
                                               int64_t lse_ld, const int32_t* cu_q, const int32_t* cu_k, int nseg,
                                               int Tq, int Tk, int heads, int head_dim, float softmax_scale,
                                               hipStream_t stream) {
  DITK_REQUIRE(v != nullptr, "ditk_flash_attn_varlen_noalloc: null tensor");
  DITK_REQUIRE(Tk >= 0 && nseg > 0 && heads > 0 && (head_dim == 64 || head_dim == 128),
               "ditk_flash_attn_varlen_noalloc: bad sizes");
  const int64_t cols = ditk_vt_columns(Tk, nseg);
  const size_t need = (size_t)heads * (size_t)head_dim * (size_t)cols * sizeof(bf16_t);
  DITK_REQUIRE(need <= kScratchBytes,
               "ditk_flash_attn_varlen_noalloc: transposed V needs %zu bytes (%d heads x %d x %lld columns), "
               "more than the %zu-byte scratch; use ditk_transpose_v + ditk_flash_attn_varlen with a caller buffer",
               need, heads, head_dim, (long long)cols, kScratchBytes);
  void* vt = scratch_ptr();
  if (vt == nullptr) return 3;
  int rc = ditk_transpose_v(v, ldv, vt, cols, Tk, heads, head_dim, cu_k, nseg, stream);
  if (rc) return rc;
  return ditk_flash_attn_varlen(q, ldq, k, ldk, vt, cols, o, ldo, lse, lse_ld, cu_q, cu_k, nseg, Tq, heads,
                                head_dim, softmax_scale, stream);
}
