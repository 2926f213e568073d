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
// Per workgroup: NW waves x QB*32 queries of one (segment, head) (defaults 8 x 32:
// two waves per SIMD, so one wave's softmax overlaps the other's MFMAs); K/Vt
// tiles of 64 keys are staged through LDS by direct global->LDS DMA (three K
// stages, two Vt stages).  Each wave computes
//   S^T = K Q^T        (A = K rows from LDS, B = Q held in registers)
//   P^T = exp2(S^T * scale*log2e - m)   (online softmax, fp32)
//   O^T += Vt P^T      (A = Vt rows from LDS, B = P^T straight from registers)
// with v_mfma_f32_32x32x16_bf16.  The K rows fed to the first MFMA are permuted
// (kperm) so that the S^T accumulator registers of each lane are exactly the
// B-operand layout of the second MFMA: no shuffles between the two products.
// Each lane owns one query of each 32-query tile, so softmax statistics are
// per-lane scalars combined across the two half-waves with one shuffle.  The
// running max is raised lazily (see rescale_tile), so the common path per score
// is one fma, one exp2, half a bf16 pack and one add.
//
// Query tiles start at each segment's first query and the key loop starts at
// each segment's first key, so results are independent of packing: a request
// packed with others is bitwise equal to the same request run alone.
//
// PRE (head_dim 64 only): Q arrives multiplied by softmax_scale*log2(e) — the
// producer folds that factor into its QK-norm weight, so Q is still rounded to
// bf16 once.  The S^T accumulators then start from a register block holding -m
// instead of zero, and P = exp2(S) takes no fma: every live S register holds
// q.k*scale*log2(e) - m_run, and whenever m_run moves by d the live S registers
// and the block move by -d.
//
// JOINT (with PRE): each joint segment's rows come from two packed sources with
// the same leading dimension — row j of segment m is row cu_a[m] + j of the
// "a" operand (image tokens) while j < len_a(m), else row cu_b[m] + j - len_a(m)
// of the "b" operand (text tokens) — for Q, K and O alike, so SD3.5's image and
// text projections feed joint attention, and take its output, without a gather
// or scatter copy.  Results are bitwise those of the gathered layout.
#include <mutex>

#include "ditk_common.h"
#include "attn_d128_clobbers.h"
#include "attn_d128p_clobbers.h"
#include "attn_d64_clobbers.h"
#include "attn_d64p_clobbers.h"

namespace {

constexpr int BN = 64;        // keys per iteration
constexpr int kWaves = 8;     // waves per workgroup: two per SIMD
constexpr int kQBlocks = 1;   // 32-query blocks per wave
constexpr int kVAhead = 2;    // Vt fragments in flight ahead of the PV MFMAs
constexpr float kLazy = 8.0f;  // log2 headroom before the running max is raised
constexpr float kRescaleSum = 256.0f;  // 2^kLazy: a lane's row sum above it triggers a rescale

// S^T row m of a 32-key MFMA tile holds key kperm(m): with the D layout
// row = (v/4)*8 + (lane/32)*4 + v%4, this puts key (v/8)*16 + (lane/32)*8 + v%8
// in accumulator register v — the B-operand k-slot order of the PV product.
__device__ __forceinline__ int kperm(int m) {
  return ((m >> 4) << 4) | (((m >> 2) & 1) << 3) | (((m >> 3) & 1) << 2) | (m & 3);
}


// 16 bytes per lane, global -> LDS; the 64 lanes of the wave fill 1 KiB of LDS
// starting at the wave-uniform `lds_slot0` (lane l writes bytes l*16..l*16+15).
// Issued as inline asm on purpose: the compiler then does not track the LDS
// write, so it does not guard every later LDS read of *another* stage with a
// full vmcnt(0) (it cannot tell the runtime stage indices apart, and that wait
// would expose the prefetch's whole latency each tile).  The kernel orders the
// DMA itself: each wave waits for its own DMA (dma_wait) before the barrier
// that publishes a stage, and no stage is read before that barrier.
// The LDS address goes in M0 through the "{m0}" operand, so the compiler sets
// M0 itself and knows it is used; the s_nop is the wait state an M0 write needs
// before an LDS DMA reads it.
__device__ __forceinline__ void lds_dma16(const bf16_t* gsrc, u32x4_t* lds_slot0) {
  const uint32_t lds_addr = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4_t*)lds_slot0);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gsrc), "{m0}"(lds_addr) : "memory");
}

__device__ __forceinline__ void dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// sched_group_barrier of n VALU/TRANS instructions; n is a constant after
// unrolling, the switch turns it into the literal the builtin needs
__device__ __forceinline__ void valu_group(int n) {
  switch (n) {
#define VG(k) case k: __builtin_amdgcn_sched_group_barrier(0x402, k, 0); break;
    VG(1) VG(2) VG(3) VG(4) VG(5) VG(6) VG(7) VG(8) VG(9) VG(10) VG(11) VG(12) VG(13) VG(14) VG(15) VG(16)
#undef VG
    default: break;
  }
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
// Per workgroup: NW waves x QB*32 queries of one (segment, head); per wave and
// 64-key tile kt (steady state):
//   A: S(kt+1) = K(kt+1) Q^T on MFMA  ||  P(kt) keys 32..63 on VALU
//   B: O += Vt(kt) P(kt) on MFMA      ||  P(kt+1) keys 0..31 on VALU
// Each K / Vt fragment read from LDS feeds QB MFMAs (one per 32-query block).
// K(kt) sits in LDS stage kt % KST (kept resident for the rescale path while
// later tiles stream in), Vt(kt) in stage kt % 2.
template <int HD, int NW, int QB, bool PRE, bool JOINT>
__global__ __launch_bounds__(NW * 64, 1) void flash_fwd_kernel(
    const bf16_t* __restrict__ Q, int64_t ldq, const bf16_t* __restrict__ Kp, int64_t ldk,
    const bf16_t* __restrict__ Vt, int64_t vt_ld, int64_t vt_hs, bf16_t* __restrict__ O, int64_t ldo,
    float* __restrict__ lse, int64_t lse_ld, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ cu_k, int nseg, int heads, int tiles_bound, float scale_log2,
    const bf16_t* __restrict__ Qb, const bf16_t* __restrict__ Kb, bf16_t* __restrict__ Ob,
    const int32_t* __restrict__ cu_a, const int32_t* __restrict__ cu_b) {
  constexpr int BM = NW * QB * 32;       // queries per workgroup
  constexpr int NC = HD / 16;            // 16-wide k chunks of the head dim
  constexpr int KCH = HD / 8;            // 16-byte chunks per K row
  constexpr int DT = HD / 32;            // 32-row d tiles of O^T
  constexpr int K_LOADS = BN * KCH / 64 / NW;   // 64-slot DMA groups per wave
  constexpr int V_LOADS = HD * 8 / 64 / NW;
  static_assert(K_LOADS >= 1 && V_LOADS >= 1 && (BN * KCH / 64) % NW == 0, "tile too small for the workgroup");
  constexpr int KST = 3;  // K stages in LDS
  __shared__ u32x4_t Ks[KST][BN * KCH];
  __shared__ u32x4_t Vs[2][HD * 8];

  // XCD-aware order: hardware deals workgroup ids round-robin over 8 XCDs, so
  // give each XCD a contiguous run of (head, tile) work — neighbouring query
  // tiles of one head then share that XCD's L2 for their K/V stream.
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  const int logical = (b & 7) * (nb >> 3) + (b >> 3);
  const int head = logical / tiles_bound;
  int t = logical % tiles_bound;
  if (head >= heads) return;
  const int seg = locate_tile(cu_q, nseg, BM, t);
  if (seg < 0) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int q_end = cu_q[seg + 1];
  const int qrow0 = cu_q[seg] + t * BM + wave * (QB * 32) + l32;  // query of block qb: qrow0 + 32 * qb
  const int k_beg = cu_k[seg], k_len = cu_k[seg + 1] - k_beg;
  const int pk = padded_key_start(cu_k, seg);

  const bf16_t* Qh = Q + (int64_t)head * HD;
  const bf16_t* Kh = Kp + (int64_t)head * HD + (int64_t)k_beg * ldk;
  const bf16_t* Vh = Vt + (int64_t)head * vt_hs + pk;
  // JOINT: row j of this segment -> its row in the a or b operand
  int a0 = 0, len_a = 0, b0 = 0;
  if (JOINT) {
    a0 = cu_a[seg];
    len_a = cu_a[seg + 1] - a0;
    b0 = cu_b[seg];
  }
  auto src_row = [&](int j) -> int64_t { return j < len_a ? (int64_t)(a0 + j) : (int64_t)(b0 + j - len_a); };
  static_assert(!JOINT || PRE, "joint sources: pre-scaled kernel only");

  // ---- Q fragments (B operand of S^T): lane -> query l32 of block qb, k-slot hh*8..+8
  bf16x8_t qf[QB][NC];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      u32x4_t v = u32x4_t{0, 0, 0, 0};
      const int qrow = qrow0 + 32 * qb;
      if (qrow < q_end) {
        if (JOINT) {
          const int j = qrow - cu_q[seg];
          const bf16_t* src = (j < len_a ? Qh : Qb + (int64_t)head * HD) + src_row(j) * ldq;
          v = *reinterpret_cast<const u32x4_t*>(src + c * 16 + hh * 8);
        } else {
          v = *reinterpret_cast<const u32x4_t*>(Qh + (int64_t)qrow * ldq + c * 16 + hh * 8);
        }
      }
      qf[qb][c] = __builtin_bit_cast(bf16x8_t, v);
    }
  // consume the Q loads here, so the compiler's own vmcnt wait for them sits
  // before the key loop rather than at the first use inside it
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int c = 0; c < NC; ++c) asm volatile("" : "+v"(qf[qb][c]));

  f32x16_t o[QB][DT];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[qb][d][v] = 0.f;
  static_assert(!PRE || HD == 64, "pre-scaled Q: head_dim 64");
  constexpr float kOne = 1.0f;
  const float sc = PRE ? kOne : scale_log2;  // S -> log2 units
  float m_run[QB], l_run[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = -INFINITY;
    l_run[qb] = 0.f;
  }
  f32x16_t negm[QB];  // PRE: -m_run in every register, the S accumulators' start

  // ---- DMA (global -> LDS, 16 B per lane).  Instruction i of wave w fills
  // slots [g*64, g*64 + 64), g = i*NW + w: rows 8*(g%(rows/8)) .. +8 of chunk
  // group g/(rows/8); lane l -> row + l/8, stored chunk l%8.  The swizzle term of
  // row (8k + l/8) is ((l >> 4) + 4k) & 7, i.e. one of two per-lane values.
  // K rows past the segment end re-read its last row; Vt padding is zero.
  const int lrow = lane >> 3;
  const int lsw0 = ((lane & 7) ^ ((lane >> 4) & 7)) * 8;        // chunk offset, k even
  const int lsw1 = ((lane & 7) ^ (((lane >> 4) + 4) & 7)) * 8;  // chunk offset, k odd
  // Per-lane element offsets of each DMA instruction from the tile's uniform base
  // (32-bit: the host bounds 64 rows of K and HD rows of Vt below 2^31 elements).
  uint32_t k_off[K_LOADS], k_col[K_LOADS], v_off[V_LOADS];
  int k_row[K_LOADS];
#pragma unroll
  for (int i = 0; i < K_LOADS; ++i) {
    const int g = i * NW + wave_u;
    const int grp = g / (BN / 8), r8 = g % (BN / 8);
    k_row[i] = r8 * 8 + lrow;
    k_col[i] = (uint32_t)(grp * 64 + ((r8 & 1) ? lsw1 : lsw0));
    k_off[i] = (uint32_t)k_row[i] * (uint32_t)ldk + k_col[i];
  }
#pragma unroll
  for (int i = 0; i < V_LOADS; ++i) {
    const int g = i * NW + wave_u;
    v_off[i] = (uint32_t)(g * 8 + lrow) * (uint32_t)vt_ld + (uint32_t)((g & 1) ? lsw1 : lsw0);
  }
  auto issue_k = [&](int kt, int s) {
    const int kb = kt * BN;
    if (JOINT) {
      const bf16_t* ka = Kp + (int64_t)head * HD;
      const bf16_t* kbp = Kb + (int64_t)head * HD;
#pragma unroll
      for (int i = 0; i < K_LOADS; ++i) {
        const int j = min(kb + k_row[i], k_len - 1);
        lds_dma16((j < len_a ? ka : kbp) + src_row(j) * ldk + k_col[i], &Ks[s][(i * NW + wave_u) * 64]);
      }
      return;
    }
    const bf16_t* base = Kh + (int64_t)kb * ldk;
    if (kb + BN <= k_len) {
#pragma unroll
      for (int i = 0; i < K_LOADS; ++i) lds_dma16(base + k_off[i], &Ks[s][(i * NW + wave_u) * 64]);
    } else {
      const int last = k_len - kb - 1;
#pragma unroll
      for (int i = 0; i < K_LOADS; ++i)
        lds_dma16(base + (uint32_t)min(k_row[i], last) * (uint32_t)ldk + k_col[i], &Ks[s][(i * NW + wave_u) * 64]);
    }
  };
  auto issue_v = [&](int kt, int s) {
    const bf16_t* base = Vh + kt * BN;
#pragma unroll
    for (int i = 0; i < V_LOADS; ++i) lds_dma16(base + v_off[i], &Vs[s][(i * NW + wave_u) * 64]);
  };

  // per-lane read bases (slot units): K row kperm(l32), chunk (c%4)*2 + hh;
  // Vt row l32, chunk (kk*2 + j)*2 + hh.  Both swizzle terms are (row>>1)&7 of
  // a row whose bits 1..3 come from l32 alone.
  int kbase[4], vbase[4];
  {
    const int kr = kperm(l32), kg = (kr >> 1) & 7, vg = (l32 >> 1) & 7;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kbase[i] = kr * 8 + ((i * 2 + hh) ^ kg);
      vbase[i] = l32 * 8 + ((i * 2 + hh) ^ vg);
    }
  }
  auto k_frag = [&](int s, int c, int kk) {
    return __builtin_bit_cast(bf16x8_t, Ks[s][kbase[c & 3] + (c >> 2) * BN * 8 + kk * 256]);
  };
  auto v_frag = [&](int s, int g, int d) { return __builtin_bit_cast(bf16x8_t, Vs[s][vbase[g] + d * 256]); };

  // S^T = K(stage s) Q^T from scratch, one K chunk in flight (prologue and the
  // rare rescale path; the steady loop interleaves its own S product)
  auto compute_s = [&](int s, f32x16_t (&sacc)[QB][2]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int v = 0; v < 16; ++v) sacc[qb][kk][v] = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const bf16x8_t kf = k_frag(s, c, kk);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          sacc[qb][kk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[qb][c], sacc[qb][kk], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);  // bounded register use: one chunk in flight
    }
  };
  // row max of S^T for this lane's query of block qb, scaled to log2 units
  auto row_max = [&](const f32x16_t (&sacc)[2]) {
    float a = fmaxf(sacc[0][0], sacc[1][0]);
#pragma unroll
    for (int v = 1; v < 16; ++v) a = fmaxf(a, fmaxf(sacc[0][v], sacc[1][v]));
    return fmaxf(a, __shfl_xor(a, 32, 64)) * sc;
  };
  // P = exp2(S*c - m) as bf16 B-operand fragments for one query block; returns
  // the fp32 row sum over keys < valid (key of register v in key tile kk:
  // kk*32 + (v/8)*16 + hh*8 + v%8).
  auto softmax_p = [&](const f32x16_t (&sacc)[2], uint32_t (&pf)[2][2][4], float m, int valid) {
    const float neg_m = -m;
    float rs = 0.f;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(sacc[kk][j * 8 + 2 * e], sc, neg_m));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(sacc[kk][j * 8 + 2 * e + 1], sc, neg_m));
          pf[kk][j][e] = pack_bf2(p0, p1);
          const int key = kk * 32 + j * 16 + hh * 8 + 2 * e;
          rs += (key < valid ? p0 : 0.f) + (key + 1 < valid ? p1 : 0.f);
        }
    return rs;
  };
  // Lazy rescale.  P(kt) is first computed against the running reference m;
  // while every score stays below m + kLazy, each P <= 2^kLazy and this lane's
  // row sum over its 32 keys stays <= 32 * 2^kLazy.  A sum above 2^kLazy (or a
  // non-finite one) therefore flags every tile that might break that bound
  // (plus a few that do not): then, rarely, S(kt) is recomputed from K(kt),
  // still resident in its LDS stage, m is raised to the tile's max, O and l are
  // rescaled and P(kt) is recomputed, for all query blocks of the wave.
  auto needs_rescale = [&](const float (&rs)[QB]) {
    bool r = false;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) r |= !(rs[qb] <= kRescaleSum);
    return __any(r);
  };
  // sr holds S - bias[qb] in log2 units (bias 0: S computed from zero)
  auto rescale_from = [&](const f32x16_t (&sr)[QB][2], uint32_t (&pf)[QB][2][2][4], float (&rs)[QB], int valid,
                          const float (&bias)[QB]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const float m_new = fmaxf(m_run[qb], PRE ? row_max(sr[qb]) + bias[qb] : row_max(sr[qb]));
      const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - m_new);
      m_run[qb] = m_new;
      l_run[qb] *= alpha;
#pragma unroll
      for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[qb][d][v] *= alpha;
      rs[qb] = softmax_p(sr[qb], pf[qb], PRE ? m_run[qb] - bias[qb] : m_run[qb], valid);
    }
  };
  auto rescale_tile = [&](int kstage, uint32_t (&pf)[QB][2][2][4], float (&rs)[QB], int valid) {
    f32x16_t sr[QB][2];
    compute_s(kstage, sr);
    const float zero[QB] = {};
    rescale_from(sr, pf, rs, valid, zero);
  };
  auto set_negm = [&]() {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int v = 0; v < 16; ++v) negm[qb][v] = -m_run[qb];
  };
  // PRE: move the live S registers to a new reference m (after m_run rose from m_old)
  auto rebias = [&](f32x16_t (&s)[QB][2], const float (&m_old)[QB]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const float d = m_run[qb] - m_old[qb];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int v = 0; v < 16; ++v) s[qb][kk][v] -= d;
    }
    set_negm();
  };
  auto pv = [&](int s, const uint32_t (&pf)[QB][2][2][4]) {
#pragma unroll
    for (int g = 0; g < 4; ++g)  // g = kk * 2 + j
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const bf16x8_t v8 = v_frag(s, g, d);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const uint32_t* p = pf[qb][g >> 1][g & 1];
          const u32x4_t p4 = u32x4_t{p[0], p[1], p[2], p[3]};
          o[qb][d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v8, __builtin_bit_cast(bf16x8_t, p4), o[qb][d], 0, 0, 0);
        }
      }
  };
  // keep packed P in registers where it is made: otherwise the packing sinks
  // below the rescale branch and the fp32 values stay live across it
  auto pin = [&](uint32_t (&pf)[QB][2][2][4]) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) asm volatile("" : "+v"(pf[qb][kk][j][e]));
  };

  // Keys past the segment end are clamped duplicates of its last key: they
  // cannot raise a row max, their Vt columns are zero, and only the final
  // tile's row sum has to skip them.
  const int nkt = (k_len + BN - 1) / BN;
  f32x16_t s_next[QB][2];
  // last tile: keys past the segment end are masked out of the row sum
  auto last = [&](const f32x16_t (&s)[QB][2]) {
    const int valid = k_len - (nkt - 1) * BN;
    uint32_t pf[QB][2][2][4];
    float rs[QB], bias[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      bias[qb] = PRE ? m_run[qb] : 0.f;
      rs[qb] = softmax_p(s[qb], pf[qb], PRE ? 0.f : m_run[qb], valid);
    }
    if (needs_rescale(rs)) rescale_from(s, pf, rs, valid, bias);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) l_run[qb] += rs[qb];
    pv((nkt - 1) & 1, pf);
  };
  // K DMA runs two tiles ahead through three stages, Vt one tile ahead through two.
  if (nkt > 0) {
    issue_k(0, 0);
    dma_wait();
    __syncthreads();
    compute_s(0, s_next);
    if (nkt > 1) issue_k(1, 1);
    issue_v(0, 0);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) m_run[qb] = row_max(s_next[qb]);  // exact max of the first tile
    if (PRE) {
      const float zero[QB] = {};
      rebias(s_next, zero);  // S(0) - m, and the -m block
    }
    dma_wait();
    __syncthreads();
  }
  // Split interleave: the 16 score pairs of a tile are spread evenly over both
  // MFMA phases of the wave.  Per tile kt:
  //   phase 1: S(kt+1) = K(kt+1) Q^T   ||  P(kt) keys 32..63
  //   (rescale check on all 64 keys of P(kt))
  //   phase 2: O += Vt(kt) P(kt)       ||  P(kt+1) keys 0..31
  // One check per tile, on the lane's row sum over both halves, before any of
  // P(kt) reaches O: it flags every tile with a score above m + kLazy (that
  // score alone makes the sum exceed 2^kLazy), and the rescale redoes the
  // whole tile from K(kt), still resident in LDS.  Keys 0..31 of P(kt+1) are
  // computed against the running m and checked with the rest of tile kt+1.
  auto pair_at = [&](const f32x16_t (&s)[QB][2], uint32_t (&pf)[QB][2][2][4], float (&rs)[QB], int qb,
                     int kk, int r) {
    const int j = r >> 2, e = r & 3;
    const float p0 = PRE ? __builtin_amdgcn_exp2f(s[qb][kk][j * 8 + 2 * e])
                         : __builtin_amdgcn_exp2f(fmaf(s[qb][kk][j * 8 + 2 * e], scale_log2, -m_run[qb]));
    const float p1 = PRE ? __builtin_amdgcn_exp2f(s[qb][kk][j * 8 + 2 * e + 1])
                         : __builtin_amdgcn_exp2f(fmaf(s[qb][kk][j * 8 + 2 * e + 1], scale_log2, -m_run[qb]));
    pf[qb][kk][j][e] = pack_bf2(p0, p1);
    rs[qb] += p0 + p1;
  };
  // A pair is issued in two halves: (2 fma, 2 exp2) and (pack, 2 add), in the
  // item order a0 a1 b0 a2 b1 ... a(n-1) b(n-2) b(n-1), so MFMAs sit between
  // each exp2 and its first use instead of a wait.
  auto item = [](int k, int n, int& pi) {  // 0: exp half of pair pi, 1: pack half
    if (k == 0) { pi = 0; return 0; }
    if (k == 2 * n - 1) { pi = n - 1; return 1; }
    if (k & 1) { pi = (k + 1) / 2; return 0; }
    pi = k / 2 - 1;
    return 1;
  };
  auto pair_a = [&](const f32x16_t (&s)[QB][2], float (&ph)[2], int qb, int kk, int r) {
    const int j = r >> 2, e = r & 3;
    if (PRE) {
      ph[0] = __builtin_amdgcn_exp2f(s[qb][kk][j * 8 + 2 * e]);
      ph[1] = __builtin_amdgcn_exp2f(s[qb][kk][j * 8 + 2 * e + 1]);
    } else {
      ph[0] = __builtin_amdgcn_exp2f(fmaf(s[qb][kk][j * 8 + 2 * e], scale_log2, -m_run[qb]));
      ph[1] = __builtin_amdgcn_exp2f(fmaf(s[qb][kk][j * 8 + 2 * e + 1], scale_log2, -m_run[qb]));
    }
  };
  auto pair_b = [&](uint32_t (&pf)[QB][2][2][4], float (&rs)[QB], const float (&ph)[2], int qb, int kk, int r) {
    pf[qb][kk][r >> 2][r & 3] = pack_bf2(ph[0], ph[1]);
    rs[qb] += ph[0] + ph[1];
  };
  // the items of slot t (of `slots`) over n pairs, and their VALU op count
  auto slot_items = [&](int t, int slots, int n, const f32x16_t (&s)[QB][2], uint32_t (&pf)[QB][2][2][4],
                        float (&rs)[QB], float (&ph)[8 * QB][2], int kk) {
#pragma unroll
    for (int k = 0; k < 2 * n; ++k)
      if ((k * slots) / (2 * n) == t) {
        int pi;
        if (item(k, n, pi) == 0) pair_a(s, ph[pi], pi / 8, kk, pi % 8);
        else pair_b(pf, rs, ph[pi], pi / 8, kk, pi % 8);
      }
  };
  auto slot_ops = [&](int t, int slots, int n) {
    int ops = 0;
    for (int k = 0; k < 2 * n; ++k)
      if ((k * slots) / (2 * n) == t) {
        int pi;
        ops += item(k, n, pi) == 0 ? (PRE ? 2 : 4) : 3;
      }
    return ops;
  };
  auto steady_split = [&](int kt, f32x16_t (&s_cur)[QB][2], f32x16_t (&s_nxt)[QB][2],
                          uint32_t (&pf_cur)[QB][2][2][4], uint32_t (&pf_nxt)[QB][2][2][4],
                          float (&rs0_cur)[QB], float (&rs0_nxt)[QB]) {
    const int knxt = (kt + 1) % KST, vcur = kt & 1;
    if (kt + 2 < nkt) issue_k(kt + 2, (kt + 2) % KST);
    issue_v(kt + 1, vcur ^ 1);
    float rs1[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) rs1[qb] = 0.f;
    // phase 1: 2*NC MFMA slots of QB MFMAs, 8*QB pairs of keys 32..63
    {
      constexpr int SLOTS = 2 * NC;
      float ph1[8 * QB][2];
      bf16x8_t kf[2][2];
      kf[0][0] = k_frag(knxt, 0, 0);
      kf[0][1] = k_frag(knxt, 0, 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int cb = c & 1;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int slot = c * 2 + kk;
#pragma unroll
          for (int qb = 0; qb < QB; ++qb)
            s_nxt[qb][kk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                kf[cb][kk], qf[qb][c], c == 0 ? (PRE ? negm[qb] : f32x16_t{}) : s_nxt[qb][kk], 0, 0, 0);
          slot_items(slot, SLOTS, 8 * QB, s_cur, pf_cur, rs1, ph1, 1);
        }
        if (c + 1 < NC) {
          kf[cb ^ 1][0] = k_frag(knxt, c + 1, 0);
          kf[cb ^ 1][1] = k_frag(knxt, c + 1, 1);
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int slot = c * 2 + kk;
          __builtin_amdgcn_sched_group_barrier(0x008, QB, 0);
          if (kk == 0 && c + 1 < NC) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          valu_group(slot_ops(slot, SLOTS, 8 * QB));
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    pin(pf_cur);
    float rsum[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) rsum[qb] = rs0_cur[qb] + rs1[qb];
    if (needs_rescale(rsum)) {
      // P(kt) keys 0..31 are not in O yet either: the whole tile is redone from
      // K(kt), still resident, so S(kt) keys 0..31 need not stay in registers
      float m_old[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) m_old[qb] = m_run[qb];
      rescale_tile(kt % KST, pf_cur, rs1, BN);
      if (PRE) rebias(s_nxt, m_old);  // S(kt+1) was started from the old -m
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) rs0_cur[qb] = 0.f;
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      l_run[qb] += rs0_cur[qb] + rs1[qb];
      rs0_nxt[qb] = 0.f;
    }
    // phase 2: 4*DT MFMA slots (one Vt fragment, QB MFMAs each), 8*QB pairs of
    // keys 0..31 of the next tile; Vt fragments read one slot ahead
    {
      constexpr int SLOTS = 4 * DT;
      float ph2[8 * QB][2];
      constexpr int VA = kVAhead;  // Vt fragments in flight
      bf16x8_t vb[VA + 1];
#pragma unroll
      for (int t = 0; t < VA; ++t) vb[t] = v_frag(vcur, t / DT, t % DT);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < SLOTS; ++t) {
        const int g = t / DT, d = t % DT;
        if (t + VA < SLOTS) vb[(t + VA) % (VA + 1)] = v_frag(vcur, (t + VA) / DT, (t + VA) % DT);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const uint32_t* p = pf_cur[qb][g >> 1][g & 1];
          const u32x4_t p4 = u32x4_t{p[0], p[1], p[2], p[3]};
          o[qb][d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb[t % (VA + 1)], __builtin_bit_cast(bf16x8_t, p4), o[qb][d], 0, 0, 0);
        }
        slot_items(t, SLOTS, 8 * QB, s_nxt, pf_nxt, rs0_nxt, ph2, 0);
        if (t + VA < SLOTS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, QB, 0);
        valu_group(slot_ops(t, SLOTS, 8 * QB));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    pin(pf_nxt);
    dma_wait();
    __syncthreads();
  };
  {
    f32x16_t (&sa)[QB][2] = s_next;
    f32x16_t sb[QB][2];
    uint32_t pfa[QB][2][2][4], pfb[QB][2][2][4];
    float rsa[QB], rsb[QB];
    if (nkt > 1) {  // keys 0..31 of tile 0 against its exact max: no check needed
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        rsa[qb] = 0.f;
#pragma unroll
        for (int r = 0; r < 8; ++r) pair_at(sa, pfa, rsa, qb, 0, r);
      }
    }
    int kt = 0;
    for (; kt + 2 < nkt; kt += 2) {
      steady_split(kt, sa, sb, pfa, pfb, rsa, rsb);
      steady_split(kt + 1, sb, sa, pfb, pfa, rsb, rsa);
    }
    // the last tile is redone from its scores with the key mask
    if (kt + 1 < nkt) {
      steady_split(kt, sa, sb, pfa, pfb, rsa, rsb);
      last(sb);
    } else if (nkt > 0) {
      last(sa);
    }
  }

  // ---- normalise and store
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float l = l_run[qb] + __shfl_xor(l_run[qb], 32, 64);
    const int qrow = qrow0 + 32 * qb;
    if (qrow < q_end) {
      const float inv = (l > 0.f) ? 1.f / l : 0.f;
      bf16_t* orow = O + (int64_t)qrow * ldo + (int64_t)head * HD;
      if (JOINT) {
        const int j = qrow - cu_q[seg];
        orow = (j < len_a ? O : Ob) + src_row(j) * ldo + (int64_t)head * HD;
      }
#pragma unroll
      for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int dd = d * 32 + g * 8 + hh * 4;
          u32x2_t w = u32x2_t{pack_bf2(o[qb][d][g * 4 + 0] * inv, o[qb][d][g * 4 + 1] * inv),
                              pack_bf2(o[qb][d][g * 4 + 2] * inv, o[qb][d][g * 4 + 3] * inv)};
          *reinterpret_cast<u32x2_t*>(orow + dd) = w;
        }
      if (lse != nullptr && hh == 0)
        lse[(int64_t)head * lse_ld + qrow] = (l > 0.f) ? (m_run[qb] + log2f(l)) * 0.6931471805599453f : -INFINITY;
    }
  }
}

// head_dim 128 or 64, 64 queries per wave (two 32-query blocks), one wave per
// SIMD: four waves and 256 queries per workgroup.  The C++ side locates the work
// item and computes per-lane addresses; the body is generated assembly
// (gen_attn.py -> attn_d128_body.inc / attn_d64_body.inc) with its registers
// placed by hand: O^T and Q in AGPRs, S^T and P in VGPRs, so that the whole
// working set stays in registers.  Same arithmetic, same order of every sum and
// the same lazy-rescale rule as flash_fwd_kernel, per score.
#define DITK_ATTN_ASM_OPERANDS                                                                                      \
  [qbase] "s"(su64(qbase)), [qoff0] "v"(qoff0), [qoff1] "v"(qoff1), [kdma_lo] "s"(su((uint32_t)kdma)),            \
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
      [xaddr] "v"(xaddr), [hh8] "v"(hh8), [lane] "v"(lanev), [qrow0] "v"(qrow0), [qrow1] "v"(qrow1)
// Pre-scaled q: the body's -m blocks take 32 more VGPRs, so the per-lane values
// it reads only outside the key loop arrive in AGPRs
#define DITK_ATTN_ASM_OPERANDS_PRE                                                                                  \
  [qbase] "s"(su64(qbase)), [qoff0] "a"(qoff0), [qoff1] "a"(qoff1), [kdma_lo] "s"(su((uint32_t)kdma)),            \
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
      [xaddr] "a"(xaddr), [hh8] "a"(hh8), [lane] "a"(lanev), [qrow0] "a"(qrow0), [qrow1] "a"(qrow1)
constexpr int kXcdChunk = 32;  // work items per XCD chunk (one per CU of an XCD)
template <int HD, bool PRE>
__global__ __launch_bounds__(256, 1) void flash_fwd_asm(
    const bf16_t* __restrict__ Q, int64_t ldq, const bf16_t* __restrict__ Kp, int64_t ldk,
    const bf16_t* __restrict__ Vt, int64_t vt_ld, int64_t vt_hs, bf16_t* __restrict__ O, int64_t ldo,
    float* __restrict__ lse, int64_t lse_ld, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ cu_k, int nseg, int heads, int np, float scale_log2) {
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
  // Q rows past the segment end read its last row (their outputs are not stored)
  const uint64_t qbase = (uint64_t)(uintptr_t)(Q + (int64_t)head * HD);
  const uint32_t qoff0 = (uint32_t)((int64_t)min(qrow0, q_end - 1) * ldq * 2 + hh * 16);
  const uint32_t qoff1 = (uint32_t)((int64_t)min(qrow1, q_end - 1) * ldq * 2 + hh * 16);
  const uint64_t kdma = (uint64_t)(uintptr_t)(Kp + (int64_t)head * HD + (int64_t)k_beg * ldk);
  const uint64_t vdma = (uint64_t)(uintptr_t)(Vt + (int64_t)head * vt_hs + pk);
  const uint32_t ktile = (uint32_t)(BN * ldk * 2);
  const uint32_t ldkb = (uint32_t)(ldk * 2);
  // LDS read bases (bytes within a stage), as flash_fwd_kernel's kbase / vbase
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
    voff[i] = (uint32_t)((int64_t)(g * 8 + lrow) * vt_ld + ((g & 1) ? lsw1 : lsw0)) * 2;
  }
  const uint32_t wave1k = (uint32_t)wave_u * 1024u;
  const uint32_t xaddr = (uint32_t)((lane ^ 32) * 4);
  const uint32_t hh8 = (uint32_t)(hh * 8);
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
  constexpr int PITCH = HD + 2;  // u16 pitch: odd word stride spreads column reads over banks
  __shared__ bf16_t tile[BN * PITCH];
  int t = blockIdx.x;
  const int head = blockIdx.y;
  const int seg = locate_tile(cu, nseg, BN, t);
  if (seg < 0) return;
  const int k0 = cu[seg] + t * BN;
  const int k_end = cu[seg + 1];
  const int col0 = padded_key_start(cu, seg) + t * BN;
  const bf16_t* Vh = V + (int64_t)head * HD;
  constexpr int CH = HD / 8;
  for (int idx = threadIdx.x; idx < BN * CH; idx += 256) {
    int r = idx / CH, ch = idx % CH;
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
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      tile[r * PITCH + ch * 8 + 2 * i] = (bf16_t)(v[i] & 0xffffu);
      tile[r * PITCH + ch * 8 + 2 * i + 1] = (bf16_t)(v[i] >> 16);
    }
  }
  __syncthreads();
  bf16_t* out = Vt + (int64_t)head * vt_hs + col0;
  for (int idx = threadIdx.x; idx < HD * (BN / 8); idx += 256) {
    int d = idx >> 3, kc = idx & 7;
    u32x4_t w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)tile[(kc * 8 + 2 * i) * PITCH + d] | ((uint32_t)tile[(kc * 8 + 2 * i + 1) * PITCH + d] << 16);
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
  DITK_REQUIRE(v && vt && cu_k, "ditk_transpose_v: null tensor");
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
  DITK_REQUIRE(q && k && vt && o && cu_q && cu_k, "ditk_flash_attn_varlen: null tensor");
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
  auto run = [&](auto kernel, int bm, int threads) -> int {
    const int tiles_bound = (Tq + bm - 1) / bm + nseg;
    int64_t nblocks = (int64_t)tiles_bound * heads;
    nblocks = (nblocks + 7) / 8 * 8;
    DITK_REQUIRE(nblocks < (1ll << 31), "ditk_flash_attn_varlen: grid too large");
    kernel<<<(unsigned)nblocks, threads, 0, stream>>>((const bf16_t*)q, ldq, (const bf16_t*)k, ldk,
                                                      (const bf16_t*)vt, vt_ld, hs, (bf16_t*)o, ldo, lse, lse_ld,
                                                      cu_q, cu_k, nseg, heads, tiles_bound, sl2, (const bf16_t*)qb,
                                                      (const bf16_t*)kb, (bf16_t*)ob, cu_a, cu_b);
    return 0;
  };
  int rc;
  if (joint)
    rc = run(flash_fwd_kernel<64, kWaves, kQBlocks, true, true>, kWaves * kQBlocks * 32, kWaves * 64);
  else {
    // one wave per SIMD, 64 queries per wave: generated-assembly body
    DITK_REQUIRE((int64_t)Tq * ldq * 2 < (1ll << 32) && ldk < (1ll << 23) && vt_ld < (1ll << 23),
                 "ditk_flash_attn_varlen: tensor too large for 32-bit lane offsets");
    // passes per work item: several query tiles per workgroup when the segments
    // have few keys (vt_ld / nseg bounds the mean key count from above), so the
    // next tile's loads hide under the current one's last key tile, as long as
    // the items still fill the CUs at least twice over (512 items at 4 tiles each)
    const int np = (vt_ld / nseg <= 2048 && (int64_t)((Tq + 255) / 256) * heads >= 2048) ? 4 : 1;
    const int tiles_bound = ((Tq + 255) / 256 + nseg + np - 1) / np + nseg;
    int64_t nblocks = (int64_t)tiles_bound * heads;
    nblocks = (nblocks + 8 * kXcdChunk - 1) / (8 * kXcdChunk) * (8 * kXcdChunk);
    DITK_REQUIRE(nblocks < (1ll << 31), "ditk_flash_attn_varlen: grid too large");
    auto kern = head_dim == 128 ? (pre ? flash_fwd_asm<128, true> : flash_fwd_asm<128, false>)
                                : (pre ? flash_fwd_asm<64, true> : flash_fwd_asm<64, false>);
    kern<<<(unsigned)nblocks, 256, 0, stream>>>((const bf16_t*)q, ldq, (const bf16_t*)k, ldk, (const bf16_t*)vt,
                                                vt_ld, hs, (bf16_t*)o, ldo, lse, lse_ld, cu_q, cu_k, nseg, heads,
                                                np, sl2);
    rc = 0;
  }
  if (rc) return rc;
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
