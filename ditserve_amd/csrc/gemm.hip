// bf16 MFMA GEMM for the DiT projections, with fused epilogues.
//
//   C[m, n] = epilogue( sum_k A[m, k] * W[n, k] + bias[n] )
//
// A is the token-major activation [M, K]; W is an nn.Linear weight [N, K]; both
// are K-contiguous, which is what the MFMA operands want (each lane feeds 8
// consecutive k values).  The kernel computes C^T tiles: the MFMA "A" operand
// is a 16-row slice of W and the "B" operand a 16-token slice of the
// activation, so every lane ends up owning one token and 4 consecutive output
// features per accumulator tile -> 8-byte row-major staging writes.
//
// Tiling (gfx950, v_mfma_f32_16x16x32_bf16, which draws less power per FLOP
// than the 32x32x16 form): a 512-thread workgroup computes a 256 (tokens) x 256
// (features) tile as 2 x 4 waves of 128 tokens x 64 features (4 x 8
// accumulator tiles of 16 x 16 per wave), two waves per SIMD so one wave's
// MFMAs issue while the other waits on its DMA or LDS reads.  K advances
// through 128 KiB of LDS stages filled by direct global->LDS DMA (no register
// staging): two stages of 64 k when K % 64 == 0, else four of 32 k.
//
// The k-loop order is fixed and there is no split-K, so every output element is
// computed the same way whatever M is and wherever its row sits: packed and
// per-request projections agree bitwise.
#include <atomic>

#include "ditk_common.h"
#include "gemm_l4_clobbers.h"

namespace {

enum Epilogue : int {
  EPI_BIAS = 0,      // bf16(acc + b)
  EPI_GELU = 1,      // bf16(gelu_tanh(bf16(acc + b)))
  EPI_GATE_RES = 2,  // bf16(R + bf16(acc + b) * gate[seg, n])   (fp32 math)
  EPI_RES = 3,       // bf16(R + bf16(acc + b))
  EPI_F32 = 4,       // fp32(acc + b)
  EPI_SILU = 5,      // bf16(silu(bf16(acc + b)))
};

// Workgroup tile configurations.  A wave computes WTM tokens x 64 features (the
// epilogue staging swizzle below assumes 64 features); the GW = WM x WN waves of
// a workgroup are laid out WM along tokens and WN along features.
//   TILE_LARGE  256 x 256, 8 waves of 128 x 64, 128 KiB of LDS stages, one
//               workgroup per CU (two waves per SIMD).
//   TILE_SMALL   64 x 128, 4 waves of 32 x 64, 72 KiB, two workgroups per CU:
//               for GEMMs whose large tiles would leave CUs idle (the few hundred
//               text rows of a step, two-row conditioning projections).
// Both run the same MFMA (W rows as the A operand) over the same k-chunk order
// with the same epilogue arithmetic, so an output element is bitwise the same
// whichever tile computed it.
enum TileCfg : int { TILE_LARGE = 0, TILE_SMALL = 1 };
template <int T> struct Tile;
template <> struct Tile<TILE_LARGE> {
  static constexpr int GBM = 256, GBN = 256, WM = 2, WN = 4, LDS_BYTES = 128 * 1024, WAVES_PER_EU = 1;
};
template <> struct Tile<TILE_SMALL> {
  static constexpr int GBM = 64, GBN = 128, WM = 2, WN = 2, LDS_BYTES = 72 * 1024, WAVES_PER_EU = 2;
};

// k-stage geometry for BK k values per stage (BK = 64 when K allows, else 32)
template <int BK, int T>
struct Stages {
  static constexpr int GBM = Tile<T>::GBM;            // tokens per workgroup tile
  static constexpr int GBN = Tile<T>::GBN;            // features per workgroup tile
  static constexpr int GW = Tile<T>::WM * Tile<T>::WN;  // waves per workgroup
  static constexpr int WTM = GBM / Tile<T>::WM;       // tokens per wave tile
  static constexpr int WTN = GBN / Tile<T>::WN;       // features per wave tile
  static constexpr int GBK = BK;
  static constexpr int NCH = BK / 32;                 // 32-k MFMA chunks per stage
  static constexpr int CPRW = BK / 8;                 // 16-byte chunks per LDS row
  static constexpr int RPG = 64 / CPRW;               // rows filled by one DMA instruction (1 KiB)
  static constexpr int DPW_A = GBM / RPG / GW;        // A DMA instructions per wave and stage
  static constexpr int DPW_W = GBN / RPG / GW;        // W DMA instructions per wave and stage
  static constexpr int ND = DPW_A + DPW_W;            // DMA instructions per wave and stage
  static constexpr int NSTAGE = Tile<T>::LDS_BYTES / ((GBM + GBN) * BK * 2);
  static_assert(WTN == 64 && DPW_A >= 1 && DPW_W >= DPW_A && DPW_A * GW * RPG == GBM &&
                    DPW_W * GW * RPG == GBN && (BK == 32 || BK == 64) && NSTAGE >= 2 &&
                    GW * WTM * WTN * 2 <= Tile<T>::LDS_BYTES,
                "tile configuration");
  // LDS stage layout (A and W alike): row r of BK k-values = CPRW chunks of
  // 16 B, slot(r, u) = r*CPRW + (u ^ swz(r)).  A DMA instruction fills 64
  // contiguous slots (RPG whole rows); 16 consecutive lanes reading chunk u of
  // 16 consecutive rows hit 16 distinct 16-byte bank groups.
  static __device__ __forceinline__ int swz(int r) { return CPRW == 4 ? (r >> 2) & 3 : (r >> 1) & 7; }
  // wait until at most `stages` DMA stages (ND instructions each) of this wave are in flight
  static __device__ __forceinline__ void dma_wait(int stages) {
    constexpr int P = ND;
    if (stages >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * P) : "memory");
    else if (stages == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(P) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
};

// Tile order: groups of `group_m` m-tiles walked m-fastest within the group, so
// the tiles running together share A rows and W rows in L2.  Chosen per shape
// (measured on the block GEMMs, same box): long K favours narrow groups
// (ffn-down: 1.39 ms at 1 vs 1.46 at 8), many n-tiles favour 4 (ffn-up: 1.58 vs
// 1.73), the rest 8.  The order does not change any result.
int gemm_group_m(int K, int tiles_n) { return K >= 4096 ? 1 : (tiles_n >= 24 ? 4 : 8); }

// 16 bytes per lane, global -> LDS; the wave's 64 lanes fill 1 KiB starting at
// the wave-uniform lds_slot0 (lane l writes bytes 16l .. 16l+15).
__device__ __forceinline__ void lds_dma16(const bf16_t* gsrc, u32x4_t* lds_slot0) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)gsrc,
                                   (__attribute__((address_space(3))) void*)lds_slot0, 16, 0, 0);
}
// Per 32 k a wave reads 4 feature fragments (double-buffered) and 8 token
// fragments (single-buffered: token fragment j of the next chunk is read right
// after the 4 MFMAs that use fragment j of this one).  Accumulator lane layout:
// features f = i*16 + 4*(lane/16) + e, token t = j*16 + lane % 16 of the wave
// tile.  The bias is loaded after the k loop (holding it through the loop would
// spill).
template <int EPI, int BK, int T>
__global__ __launch_bounds__(Tile<T>::WM * Tile<T>::WN * 64, Tile<T>::WAVES_PER_EU) void gemm_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ W, int64_t ldw,
    const float* __restrict__ bias, void* __restrict__ Cv, int64_t ldc, int M, int N, int K,
    const bf16_t* R, int64_t ldr, const float* __restrict__ gate, int64_t gate_stride,
    const int32_t* __restrict__ cu, int nseg, int tiles_m, int tiles_n, int group_m, int row_base) {
  using S = Stages<BK, T>;
  constexpr int GBM = S::GBM, GBN = S::GBN, GW = S::GW, WTM = S::WTM, WTN = S::WTN;
  constexpr int CPRW = S::CPRW, RPG = S::RPG, NSTAGE = S::NSTAGE, DPW_A = S::DPW_A, DPW_W = S::DPW_W;
  constexpr int ND = S::ND, NCH = S::NCH;
  constexpr int FI = WTN / 16, FJ = WTM / 16;  // feature / token fragments per wave (4; 8 or 2)
  __shared__ u32x4_t lds[NSTAGE * (GBM + GBN) * CPRW];
  auto As = [&](int s) { return lds + s * (GBM * CPRW); };
  auto Ws = [&](int s) { return lds + NSTAGE * GBM * CPRW + s * (GBN * CPRW); };

  const int nb = gridDim.x, b = blockIdx.x;
  const int L = (b & 7) * (nb >> 3) + (b >> 3);
  if (L >= tiles_m * tiles_n) return;
  const int group = L / (group_m * tiles_n);
  const int first_m = group * group_m;
  const int gm = min(group_m, tiles_m - first_m);
  const int pid = L % (group_m * tiles_n);
  const int mt = first_m + pid % gm, nt = pid / gm;
  const int m0 = mt * GBM, n0 = nt * GBN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ql = lane & 15, g = lane >> 4;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int wm = wave_u % Tile<T>::WM, wn = wave_u / Tile<T>::WM;
  const int a_row0 = wm * WTM, w_row0 = wn * WTN;

  const bf16_t* Ablk = A + (int64_t)m0 * lda;
  const bf16_t* Wblk = W + (int64_t)n0 * ldw;
  uint32_t a_off[DPW_A], w_off[DPW_W];
#pragma unroll
  for (int i = 0; i < DPW_W; ++i) {
    const int gi = i * GW + wave_u;
    const int row = gi * RPG + lane / CPRW;
    const int ksw = ((lane % CPRW) ^ S::swz(row)) * 8;
    if (i < DPW_A) a_off[i] = (uint32_t)(min(row, M - 1 - m0) * lda + ksw);
    w_off[i] = (uint32_t)(min(row, N - 1 - n0) * ldw + ksw);
  }
  // DMA instruction d of a stage: A and W alternate while both have
  // instructions left, then the remaining W ones
  auto dma_one = [&](int kt, int d) {
    const int s = kt % NSTAGE;
    if (d < 2 * DPW_A) {
      const int i = d >> 1, gi = i * GW + wave_u;
      if ((d & 1) == 0) lds_dma16(Ablk + kt * BK + a_off[i], &As(s)[gi * 64]);
      else lds_dma16(Wblk + kt * BK + w_off[i], &Ws(s)[gi * 64]);
    } else {
      const int i = d - DPW_A, gi = i * GW + wave_u;
      lds_dma16(Wblk + kt * BK + w_off[i], &Ws(s)[gi * 64]);
    }
  };
  auto issue = [&](int kt) {
#pragma unroll
    for (int d = 0; d < ND; ++d) dma_one(kt, d);
  };

  // operand read base of chunk c: row x*16 + ql, 16-byte chunk c*4 + g (the
  // stage swizzle of row x*16 + ql depends on ql only)
  int rbase[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) rbase[c] = ql * CPRW + ((c * 4 + g) ^ S::swz(ql));

  f32x4_t bvec[FI];
  auto load_bias = [&]() {
#pragma unroll
    for (int i = 0; i < FI; ++i)
      bvec[i] = bias != nullptr ? *reinterpret_cast<const f32x4_t*>(bias + min(n0 + w_row0 + i * 16 + 4 * g, N - 4))
                                : f32x4_t{0.f, 0.f, 0.f, 0.f};
  };

  f32x4_t acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = K / BK;
  bf16x8_t fw[2][FI], fx[FJ];
  auto read_w = [&](int s, int c, int i, bf16x8_t (&dst)[FI]) {
    dst[i] = __builtin_bit_cast(bf16x8_t, Ws(s)[rbase[c] + (w_row0 + i * 16) * CPRW]);
  };
  auto read_x = [&](int s, int c, int j) {
    fx[j] = __builtin_bit_cast(bf16x8_t, As(s)[rbase[c] + (a_row0 + j * 16) * CPRW]);
  };
#pragma unroll
  for (int kt = 0; kt < NSTAGE; ++kt)
    if (kt < nk) issue(kt);
  S::dma_wait(min(NSTAGE - 1, nk - 1));
  __syncthreads();
#pragma unroll
  for (int i = 0; i < FI; ++i) read_w(0, 0, i, fw[0]);
#pragma unroll
  for (int j = 0; j < FJ; ++j) read_x(0, 0, j);

  auto publish = [&]() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
  };
  // group j of a chunk (operand set p for the feature fragments): the FI MFMAs of
  // token fragment j, then the reads of the next chunk (cn of stage sn): token
  // fragment j into fx[j] and this group's share of the feature fragments into
  // set p^1 (one every other group when FJ = 8, two per group when FJ = 2);
  // and DMA instructions j, j + FJ, ... of stage kd
  auto step = [&](int j, int p, int sn, int cn, int kd, bool reads, bool dmas) {
#pragma unroll
    for (int i = 0; i < FI; ++i)
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fw[p][i], fx[j], acc[i][j], 0, 0, 0);
    if (reads) {
      read_x(sn, cn, j);
      if (FJ >= FI) {
        if (j % (FJ / FI) == FJ / FI - 1) read_w(sn, cn, j / (FJ / FI), fw[p ^ 1]);
      } else {
#pragma unroll
        for (int i = j * (FI / FJ); i < (j + 1) * (FI / FJ); ++i) read_w(sn, cn, i, fw[p ^ 1]);
      }
    }
    if (dmas) {
#pragma unroll
      for (int d = j; d < ND; d += FJ) dma_one(kd, d);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  static_assert((FJ % FI == 0 || FI % FJ == 0) && (NCH % 2 == 0 || NCH == 1), "group layout");
  // with one chunk per stage the next stage's feature fragments land in set 1:
  // swap the two sets after each stage (4 fragments, only the 32-k stage path)
  auto rotate = [&]() {
    if (NCH % 2 == 1) {
#pragma unroll
      for (int i = 0; i < FI; ++i) {
        const bf16x8_t t = fw[0][i];
        fw[0][i] = fw[1][i];
        fw[1][i] = t;
      }
    }
  };
  int kt = 0;
  for (; kt + NSTAGE < nk; ++kt) {
    const int s = kt % NSTAGE;
#pragma unroll
    for (int c = 0; c + 1 < NCH; ++c)
#pragma unroll
      for (int j = 0; j < FJ; ++j) step(j, c & 1, s, c + 1, 0, true, false);
    S::dma_wait(NSTAGE - 2);
    publish();
#pragma unroll
    for (int j = 0; j < FJ; ++j) step(j, (NCH - 1) & 1, (kt + 1) % NSTAGE, 0, kt + NSTAGE, true, true);
    rotate();
  }
  for (; kt < nk; ++kt) {
    const int s = kt % NSTAGE;
#pragma unroll
    for (int c = 0; c + 1 < NCH; ++c)
#pragma unroll
      for (int j = 0; j < FJ; ++j) step(j, c & 1, s, c + 1, 0, true, false);
    const bool next = kt + 1 < nk;
    if (next) {
      S::dma_wait(nk - 2 - kt);
      publish();
    }
#pragma unroll
    for (int j = 0; j < FJ; ++j) step(j, (NCH - 1) & 1, (kt + 1) % NSTAGE, 0, 0, next, false);
    rotate();
  }
  __syncthreads();
  load_bias();

  if (EPI == EPI_F32) {
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      const int m = m0 + a_row0 + j * 16 + ql;
      if (m >= M) continue;
#pragma unroll
      for (int i = 0; i < FI; ++i) {
        const int n = n0 + w_row0 + i * 16 + 4 * g;
        if (n >= N) continue;
        *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(Cv) + (int64_t)m * ldc + n) = acc[i][j] + bvec[i];
      }
    }
    return;
  }
  // bf16 epilogues through a per-wave LDS tile [WTM tokens][WTN features]: 8-byte
  // unit u (features 4u..4u+3) of row t stored at u ^ (2 * ((t >> 1) & 7)), so the
  // 16 rows of one write hit distinct banks and 16-byte unit pairs stay together.
  constexpr int CPR = WTN / 8;
  constexpr int RPP = 64 / CPR;
  constexpr int NPASS = WTM / RPP;
  constexpr bool HAS_RES = EPI == EPI_GATE_RES || EPI == EPI_RES;
  const int c8 = lane % CPR;
  const int n = n0 + w_row0 + c8 * 8;
  const int mrow = m0 + a_row0 + lane / CPR;
  u32x4_t res[HAS_RES ? NPASS : 1];
  if (HAS_RES) {
#pragma unroll
    for (int r = 0; r < NPASS; ++r) {
      const int m = mrow + r * RPP;
      res[r] = (m < M && n < N) ? *reinterpret_cast<const u32x4_t*>(R + (int64_t)m * ldr + n) : u32x4_t{0, 0, 0, 0};
    }
  }
  int seg_lo = 0;
  bool one_seg = true;
  f32x4_t g0 = {0.f, 0.f, 0.f, 0.f}, g1 = {0.f, 0.f, 0.f, 0.f};
  if (EPI == EPI_GATE_RES) {
    seg_lo = find_segment(cu, nseg, row_base + m0 + a_row0);
    one_seg = seg_lo == find_segment(cu, nseg, row_base + min(m0 + a_row0 + WTM, M) - 1);
    if (one_seg && n < N) {
      const float* gp = gate + (int64_t)seg_lo * gate_stride + n;
      g0 = *reinterpret_cast<const f32x4_t*>(gp);
      g1 = *reinterpret_cast<const f32x4_t*>(gp + 4);
    }
  }
  u32x2_t* stage8 = reinterpret_cast<u32x2_t*>(lds + wave_u * (WTM * CPR));
  const u32x4_t* stage16 = lds + wave_u * (WTM * CPR);
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      const int t = j * 16 + ql;
      const int u = (i * 4 + g) ^ (2 * ((t >> 1) & 7));
      const f32x4_t y = acc[i][j] + bvec[i];
      stage8[t * (2 * CPR) + u] = u32x2_t{pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3])};
    }
  __syncthreads();
  if (n >= N) return;
#pragma unroll
  for (int r = 0; r < NPASS; ++r) {
    const int t = r * RPP + lane / CPR;
    const int m = mrow + r * RPP;
    if (m >= M) continue;
    u32x4_t v = stage16[t * CPR + (c8 ^ ((t >> 1) & 7))];
    if (EPI != EPI_BIAS) {
      float x[8];
      unpack8(v, x);
      if (EPI == EPI_GELU) {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = gelu_tanh_f(x[e]);
      } else if (EPI == EPI_SILU) {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = silu_f(x[e]);
      } else {
        float rv[8];
        unpack8(res[HAS_RES ? r : 0], rv);
        if (EPI == EPI_GATE_RES) {
          f32x4_t h0 = g0, h1 = g1;
          if (!one_seg) {
            const float* gp = gate + (int64_t)find_segment(cu, nseg, row_base + m) * gate_stride + n;
            h0 = *reinterpret_cast<const f32x4_t*>(gp);
            h1 = *reinterpret_cast<const f32x4_t*>(gp + 4);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x[e] = fmaf(x[e], h0[e], rv[e]);
            x[e + 4] = fmaf(x[e + 4], h1[e], rv[e + 4]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = rv[e] + x[e];
        }
      }
      v = pack8(x);
    }
    u32x4_t* dst = reinterpret_cast<u32x4_t*>(reinterpret_cast<bf16_t*>(Cv) + (int64_t)m * ldc + n);
    // large-tile outputs (>= 16 MB) are streamed: the next kernel reads them back
    // from HBM anyway, and non-temporal stores measured 2.6-3.6% faster on the
    // K = 1536 block GEMMs (qkv, ffn up, o-proj), unchanged on ffn down
    if (T == TILE_LARGE) __builtin_nontemporal_store(v, dst);
    else *dst = v;
  }
}

// Large tiles on one wave per SIMD (every epilogue but fp32, K % 64 == 0): the
// 256 x 256 workgroup tile as four 128 x 128 wave tiles, 256 accumulators per
// wave in the AGPRs.  The k loop and the bf16 staging are generated assembly
// (gen_gemm.py -> gemm_l4_body.inc: 64-k stages through two 64 KiB LDS buffers
// filled by direct DMA, the next chunk's fragments read under the current
// MFMAs); this C++ part computes the per-lane addresses and runs the
// same epilogue arithmetic as gemm_kernel on the staged rows.  Same MFMA
// (16x16x32, W rows as the A operand), same k order, same bias add and rounding:
// bitwise equal to gemm_kernel.
// FI feature fragments of 16 per wave tile: 8 (128 x 128 wave tiles, 256 x 256
// workgroup tiles, gemm_l4_body.inc) or 6 (128 x 96, 256 x 192,
// gemm_l4w96_body.inc: for shapes whose 256-wide tiles would leave CUs idle in
// the last round).
template <int FI>
struct L4 {
  static constexpr int WTM = 128, WTN = 16 * FI, GBM = 256, GBN = 2 * WTN;
  static constexpr int BUF = (GBM + GBN) * 128;            // one 64-k stage: A rows, then W rows
  static constexpr int STG_ROW = 2 * WTN + 16;             // staging row bytes
  static constexpr int LDS_BYTES = 2 * BUF > 4 * WTM * STG_ROW ? 2 * BUF : 4 * WTM * STG_ROW;
};
#define DITK_L4_OPERANDS                                                                                        \
  [a_lo] "s"(su((uint32_t)abase)), [a_hi] "s"(su((uint32_t)(abase >> 32))), [w_lo] "s"(su((uint32_t)wbase)),   \
      [w_hi] "s"(su((uint32_t)(wbase >> 32))), [nk] "s"(su(K / 64)), [lds] "s"(su(lds0)),                       \
      [wave1k] "s"(su(wave_u * 1024u)), [rdx00] "v"(rdx[0][0]), [rdx01] "v"(rdx[0][1]), [rdx10] "v"(rdx[1][0]), \
      [rdx11] "v"(rdx[1][1]), [rdw00] "v"(rdw[0][0]), [rdw01] "v"(rdw[0][1]), [rdw10] "v"(rdw[1][0]),           \
      [rdw11] "v"(rdw[1][1]), [aoff0] "v"(aoff[0]), [aoff1] "v"(aoff[1]), [aoff2] "v"(aoff[2]),                 \
      [aoff3] "v"(aoff[3]), [aoff4] "v"(aoff[4]), [aoff5] "v"(aoff[5]), [aoff6] "v"(aoff[6]),                   \
      [aoff7] "v"(aoff[7]), [woff0] "v"(woff[0]), [woff1] "v"(woff[1]), [woff2] "v"(woff[2]),                   \
      [woff3] "v"(woff[3]), [woff4] "v"(woff[4]), [woff5] "v"(woff[5]), [woff6] "v"(woff[6]),                   \
      [woff7] "v"(woff[7]), [stg] "v"(stg), [b0] "v"(bv[0]), [b1] "v"(bv[1]), [b2] "v"(bv[2]), [b3] "v"(bv[3]),  \
      [b4] "v"(bv[4]), [b5] "v"(bv[5]), [b6] "v"(bv[6]), [b7] "v"(bv[7]), [b8] "v"(bv[8]), [b9] "v"(bv[9]),      \
      [b10] "v"(bv[10]), [b11] "v"(bv[11]), [b12] "v"(bv[12]), [b13] "v"(bv[13]), [b14] "v"(bv[14]),            \
      [b15] "v"(bv[15]), [b16] "v"(bv[16]), [b17] "v"(bv[17]), [b18] "v"(bv[18]), [b19] "v"(bv[19]),            \
      [b20] "v"(bv[20]), [b21] "v"(bv[21]), [b22] "v"(bv[22]), [b23] "v"(bv[23]), [b24] "v"(bv[24]),            \
      [b25] "v"(bv[25]), [b26] "v"(bv[26]), [b27] "v"(bv[27]), [b28] "v"(bv[28]), [b29] "v"(bv[29]),            \
      [b30] "v"(bv[30]), [b31] "v"(bv[31])
template <int EPI, int FI>
__device__ __forceinline__ void l4_tile(u32x4_t* lds, int L, const bf16_t* __restrict__ A, int64_t lda,
                                        const bf16_t* __restrict__ W, int64_t ldw, const float* __restrict__ bias,
                                        void* __restrict__ Cv, int64_t ldc, int M, int N, int K, const bf16_t* R,
                                        int64_t ldr, const float* __restrict__ gate, int64_t gate_stride,
                                        const int32_t* __restrict__ cu, int nseg, int tiles_m, int tiles_n,
                                        int group_m);
template <int EPI, int FI>
__global__ __launch_bounds__(256, 1) void gemm_kernel_l4(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ W, int64_t ldw,
    const float* __restrict__ bias, void* __restrict__ Cv, int64_t ldc, int M, int N, int K,
    const bf16_t* R, int64_t ldr, const float* __restrict__ gate, int64_t gate_stride,
    const int32_t* __restrict__ cu, int nseg, int tiles_m, int tiles_n, int group_m) {
  __shared__ u32x4_t lds[L4<FI>::LDS_BYTES / 16];
  // Persistent: XCD x (= blockIdx % 8) owns the tiles [x * per_xcd, (x + 1) *
  // per_xcd), which its workgroups take in turn (the order a one-tile-per-
  // workgroup launch would run them in), so each workgroup loads its kernel
  // arguments once and a tile's k loop starts while the previous tile's
  // stores drain.
  const int nb = gridDim.x, b = blockIdx.x;
  const int ntiles = tiles_m * tiles_n, per_xcd = (ntiles + 7) / 8;
  const int tlo = (b & 7) * per_xcd, thi = min(tlo + per_xcd, ntiles);
  for (int L = tlo + (b >> 3); L < thi; L += nb >> 3)
    l4_tile<EPI, FI>(lds, L, A, lda, W, ldw, bias, Cv, ldc, M, N, K, R, ldr, gate, gate_stride, cu, nseg, tiles_m,
                     tiles_n, group_m);
}

// One product of a paired launch (see gemm_kernel_l4_pair).
struct L4Prob {
  const bf16_t* A;
  int64_t lda;
  const bf16_t* W;
  int64_t ldw;
  const float* bias;
  void* C;
  int64_t ldc;
  const bf16_t* R;
  int64_t ldr;
  const float* gate;
  int64_t gate_stride;
  const int32_t* cu;
  int nseg, M, tiles_m, group_m;
};

// Two products of the same N, K and epilogue (their own inputs, weights, bias,
// residual, gate and segments) in one persistent launch: the tile list is the
// first product's tiles, then the second's, taken per XCD as gemm_kernel_l4
// takes one product's.  Each tile is computed exactly as a launch of its own
// product would compute it.
template <int EPI, int FI>
__global__ __launch_bounds__(256, 1) void gemm_kernel_l4_pair(L4Prob p0, L4Prob p1, int N, int K, int tiles_n) {
  __shared__ u32x4_t lds[L4<FI>::LDS_BYTES / 16];
  const int nb = gridDim.x, b = blockIdx.x;
  const int t0 = p0.tiles_m * tiles_n, ntiles = t0 + p1.tiles_m * tiles_n, per_xcd = (ntiles + 7) / 8;
  const int tlo = (b & 7) * per_xcd, thi = min(tlo + per_xcd, ntiles);
  for (int L = tlo + (b >> 3); L < thi; L += nb >> 3) {
    const bool s = L >= t0;  // wave-uniform: the fields below are scalar selects
    l4_tile<EPI, FI>(lds, s ? L - t0 : L, s ? p1.A : p0.A, s ? p1.lda : p0.lda, s ? p1.W : p0.W,
                     s ? p1.ldw : p0.ldw, s ? p1.bias : p0.bias, s ? p1.C : p0.C, s ? p1.ldc : p0.ldc,
                     s ? p1.M : p0.M, N, K, s ? p1.R : p0.R, s ? p1.ldr : p0.ldr, s ? p1.gate : p0.gate,
                     s ? p1.gate_stride : p0.gate_stride, s ? p1.cu : p0.cu, s ? p1.nseg : p0.nseg,
                     s ? p1.tiles_m : p0.tiles_m, tiles_n, s ? p1.group_m : p0.group_m);
  }
}

template <int EPI, int FI>
__device__ __forceinline__ void l4_tile(u32x4_t* lds, int L, const bf16_t* __restrict__ A, int64_t lda,
                                        const bf16_t* __restrict__ W, int64_t ldw, const float* __restrict__ bias,
                                        void* __restrict__ Cv, int64_t ldc, int M, int N, int K, const bf16_t* R,
                                        int64_t ldr, const float* __restrict__ gate, int64_t gate_stride,
                                        const int32_t* __restrict__ cu, int nseg, int tiles_m, int tiles_n,
                                        int group_m) {
  using G = L4<FI>;
  constexpr int GBM = G::GBM, GBN = G::GBN, WTM = G::WTM, WTN = G::WTN, STG_ROW = G::STG_ROW;
  const int group = L / (group_m * tiles_n);
  const int first_m = group * group_m;
  const int gm = min(group_m, tiles_m - first_m);
  const int pid = L % (group_m * tiles_n);
  const int mt = first_m + pid % gm, nt = pid / gm;
  const int m0 = mt * GBM, n0 = nt * GBN;

  // the lane's values are recomputed per tile (an opaque copy of the thread id
  // keeps them out of the registers that stay live across the k loop)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int ql = lane & 15, g = lane >> 4;
  const int wave_u = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int a_row0 = (wave_u & 1) * WTM, w_row0 = (wave_u >> 1) * WTN;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4_t*)&lds[0];
  // fragment reads of 32-k chunk c: row ql of a 16-row fragment, 16-byte unit
  // 4 c + g of its 64 k, stored at unit (4 c + g) ^ ((row >> 1) & 7) of the
  // 128-byte LDS row (as gemm_kernel's 64-k stages)
  uint32_t rdx[2][2], rdw[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const uint32_t lane_part = (uint32_t)(ql * 128 + (((c * 4 + g) ^ ((ql >> 1) & 7)) * 16));
      rdx[s][c] = lds0 + s * G::BUF + a_row0 * 128 + lane_part;
      rdw[s][c] = lds0 + s * G::BUF + GBM * 128 + w_row0 * 128 + lane_part;
    }
  // DMA instruction d of this wave fills rows 8 (4 d + wave) .. +7 (1 KiB):
  // lane l -> row l / 8, LDS unit l % 8 <- k unit (l % 8) ^ ((row >> 1) & 7)
  uint32_t aoff[8], woff[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    const int row = (d * 4 + wave_u) * 8 + lane / 8;
    const int usw = ((lane & 7) ^ ((row >> 1) & 7)) * 16;
    aoff[d] = (uint32_t)((int64_t)min(row, M - 1 - m0) * lda * 2 + usw);
    woff[d] = d < FI ? (uint32_t)((int64_t)min(row, N - 1 - n0) * ldw * 2 + usw) : 0u;
  }
  const uint32_t stg = lds0 + wave_u * (WTM * STG_ROW) + ql * STG_ROW + g * 8;
  float bv[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const f32x4_t x = bias != nullptr && i < FI
                          ? *reinterpret_cast<const f32x4_t*>(bias + min(n0 + w_row0 + i * 16 + 4 * g, N - 4))
                          : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) bv[i * 4 + e] = x[e];
  }
  auto su = [](uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); };
  const uint64_t abase = (uint64_t)(uintptr_t)(A + (int64_t)m0 * lda);
  const uint64_t wbase = (uint64_t)(uintptr_t)(W + (int64_t)n0 * ldw);
  if constexpr (FI == 8)
    asm volatile(
#include "gemm_l4_body.inc"
        : : DITK_L4_OPERANDS : DITK_GEMM_L4_CLOBBERS "scc", "memory");
  else
    asm volatile(
#include "gemm_l4w96_body.inc"
        : : DITK_L4_OPERANDS : DITK_GEMM_L4_CLOBBERS "scc", "memory");

  // epilogue on this wave's staged rows (the wave wrote them and waited for them).
  // The output (and residual) rows go through buffer descriptors whose range
  // ends at the last row of the matrix: a store past it is dropped and a load
  // returns 0, so the passes have no branches and the staged-row reads and
  // residual loads of many passes are in flight together.
  constexpr int CPR = WTN / 8;                    // 16-byte units per row (16 or 12)
  constexpr int RPP = 64 / CPR;                   // rows per pass (4 or 5; lanes past RPP * CPR idle)
  constexpr int NPASS = (WTM + RPP - 1) / RPP;
  constexpr bool HAS_RES = EPI == EPI_GATE_RES || EPI == EPI_RES;
  constexpr uint32_t kOut = 0x80000000u;          // an offset past every descriptor's range
  const int row0 = m0 + a_row0;                   // this wave tile's first row
  const int rows = max(0, min(WTM, M - row0));    // its rows inside the matrix
  const uint32_t ldc2 = (uint32_t)(ldc * 2), ldr2 = (uint32_t)(ldr * 2);
  // descriptors from wave-uniform (scalar) base addresses
  auto sptr = [&](const void* p) {
    const uint64_t x = (uint64_t)(uintptr_t)p;
    const uint64_t lo = su((uint32_t)x), hi = su((uint32_t)(x >> 32));
    return reinterpret_cast<void*>((uintptr_t)(lo | (hi << 32)));
  };
  const int rec_c = (int)su((uint32_t)rows * ldc2), rec_r = (int)su((uint32_t)rows * ldr2);
  const __amdgpu_buffer_rsrc_t cdesc = __builtin_amdgcn_make_buffer_rsrc(
      sptr(reinterpret_cast<bf16_t*>(Cv) + (int64_t)row0 * ldc + n0 + w_row0), 0, rec_c, 0x00020000);
  const __amdgpu_buffer_rsrc_t rdesc = __builtin_amdgcn_make_buffer_rsrc(
      sptr(HAS_RES ? R + (int64_t)row0 * ldr + n0 + w_row0 : nullptr), 0, HAS_RES ? rec_r : 0, 0x00020000);
  const int c8 = lane % CPR;
  const int n = n0 + w_row0 + c8 * 8;
  const bool lane_on = n < N && lane < RPP * CPR;   // lanes past N or past a pass's units store nothing
  const char* stage = reinterpret_cast<const char*>(lds) + wave_u * (WTM * STG_ROW);
  int seg_lo = 0;
  bool one_seg = true;
  f32x4_t g0 = {0.f, 0.f, 0.f, 0.f}, g1 = {0.f, 0.f, 0.f, 0.f};
  if (EPI == EPI_GATE_RES) {
    seg_lo = find_segment(cu, nseg, min(row0, M - 1));
    one_seg = seg_lo == find_segment(cu, nseg, min(row0 + WTM, M) - 1);
    if (one_seg) {
      const float* gp = gate + (int64_t)seg_lo * gate_stride + min(n, N - 8);
      g0 = *reinterpret_cast<const f32x4_t*>(gp);
      g1 = *reinterpret_cast<const f32x4_t*>(gp + 4);
    }
  }
  // every residual row is loaded first (one latency for the tile), then the
  // staged rows are read and stored in batches of RB passes
  u32x4_t res[HAS_RES ? NPASS : 1];
  if (HAS_RES) {
#pragma unroll
    for (int r = 0; r < NPASS; ++r) {
      const int t = r * RPP + lane / CPR;
      res[r] = __builtin_amdgcn_raw_buffer_load_b128(rdesc, t < rows && lane_on ? (uint32_t)t * ldr2 + c8 * 16 : kOut, 0, 0);
    }
  }
  constexpr int RB = 8;
#pragma unroll
  for (int r0 = 0; r0 < NPASS; r0 += RB) {
    u32x4_t v[RB];
    uint32_t off[RB];
#pragma unroll
    for (int q = 0; q < RB && r0 + q < NPASS; ++q) {
      const int t = (r0 + q) * RPP + lane / CPR;  // row in the wave tile
      off[q] = t < rows && lane_on ? (uint32_t)t * ldc2 + c8 * 16 : kOut;
      v[q] = *reinterpret_cast<const u32x4_t*>(stage + min(t, WTM - 1) * STG_ROW + c8 * 16);
    }
#pragma unroll
    for (int q = 0; q < RB && r0 + q < NPASS; ++q) {
      if (EPI != EPI_BIAS) {
        float x[8];
        unpack8(v[q], x);
        if (EPI == EPI_GELU) {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = gelu_tanh_f(x[e]);
        } else if (EPI == EPI_SILU) {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = silu_f(x[e]);
        } else {
          float rv[8];
          unpack8(res[HAS_RES ? r0 + q : 0], rv);
          if (EPI == EPI_GATE_RES) {
            f32x4_t h0 = g0, h1 = g1;
            if (!one_seg) {
              const int m = min(row0 + (r0 + q) * RPP + lane / CPR, M - 1);
              const float* gp = gate + (int64_t)find_segment(cu, nseg, m) * gate_stride + min(n, N - 8);
              h0 = *reinterpret_cast<const f32x4_t*>(gp);
              h1 = *reinterpret_cast<const f32x4_t*>(gp + 4);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              x[e] = fmaf(x[e], h0[e], rv[e]);
              x[e + 4] = fmaf(x[e + 4], h1[e], rv[e + 4]);
            }
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = rv[e] + x[e];
          }
        }
        v[q] = pack8(x);
      }
      __builtin_amdgcn_raw_buffer_store_b128(v[q], cdesc, off[q], 0, 2);  // non-temporal
    }
  }
}

// CUs of the current device, cached per device (callers on several host
// threads may race to fill an entry; they store the same value)
int cu_count() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int c = cached[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    int n = 0;
    c = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    cached[dev].store(c, std::memory_order_relaxed);
  }
  return c;
}
template <int EPI, int FI>
int launch_l4(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias, void* C, int64_t ldc,
              int M, int N, int K, const void* R, int64_t ldr, const float* gate, int64_t gate_stride,
              const int32_t* cu, int nseg, hipStream_t stream) {
  constexpr int GBN = L4<FI>::GBN;
  const int tiles_m = (M + 255) / 256, tiles_n = (N + GBN - 1) / GBN;
  // one persistent workgroup per CU (a multiple of 8: the same number per XCD)
  const int64_t nblocks = std::min<int64_t>(((int64_t)tiles_m * tiles_n + 7) / 8 * 8, std::max(8, cu_count() / 8 * 8));
  gemm_kernel_l4<EPI, FI><<<(unsigned)nblocks, 256, 0, stream>>>(
      (const bf16_t*)A, lda, (const bf16_t*)W, ldw, bias, C, ldc, M, N, K, (const bf16_t*)R, ldr, gate,
      gate_stride, cu, nseg, tiles_m, tiles_n, gemm_group_m(K, tiles_n));
  return ditk_check_launch("ditk_gemm");
}

template <int EPI>
int launch_l4_pair(L4Prob p0, L4Prob p1, int N, int K, hipStream_t stream) {
  const int tiles_n = (N + 255) / 256;
  p0.tiles_m = (p0.M + 255) / 256;
  p1.tiles_m = (p1.M + 255) / 256;
  p0.group_m = p1.group_m = gemm_group_m(K, tiles_n);
  const int64_t tiles = (int64_t)(p0.tiles_m + p1.tiles_m) * tiles_n;
  const int64_t nblocks = std::min<int64_t>((tiles + 7) / 8 * 8, std::max(8, cu_count() / 8 * 8));
  gemm_kernel_l4_pair<EPI, 8><<<(unsigned)nblocks, 256, 0, stream>>>(p0, p1, N, K, tiles_n);
  return ditk_check_launch("ditk_gemm_pair");
}

// The one-wave-per-SIMD kernel where it measured faster than gemm_kernel's large
// tiles (same box, Wan2.1 block shapes at M = 65520): N >= 3072 or K >= 4096
// (qkv -3.4%, ffn-up -2.9%, ffn-down -4.7%, N = 3072 SiLU -3.3%), and, since its
// workgroups are persistent, at N = K = 1536 too except with the gated residual
// (bias -4%, residual -4%; gated residual +3%, also with the gate looked up
// before the k loop).  The choice changes no result.
bool use_l4(int N, int K, int epi) {
  return K % 64 == 0 && (N >= 3072 || K >= 4096 || epi != EPI_GATE_RES);
}

// 256 x 192 tiles when they fill the GPU's CUs in fewer tile-rounds than
// 256 x 256 ones, a 192-wide tile taking 0.85 of a 256-wide one's time (measured
// 0.82-0.88 at M = 54560, K = 3072-14336: its k loop moves the same token rows
// for 3/4 of the MFMAs): e.g. M = 8192 and N = 1536 is 256 tiles = one round
// instead of 192 = one round with a quarter of the CUs idle (SD3.5: ffn-down
// -12%); N = 4608 is 768 tiles = 3 rounds instead of 576 = 2.25, so 3 (SD3.5
// qkv -16%); but M = 54560 and N = 3072 is 3424 tiles = 14 rounds instead of
// 2568 = 11 (Wan2.2-5B: ffn-down -11%, qkv -8%, o-proj -6% with 256-wide tiles).
bool use_w192(int M, int N) {
  const int64_t tm = (M + 255) / 256, ncu = cu_count();
  const int64_t r256 = (tm * ((N + 255) / 256) + ncu - 1) / ncu, r192 = (tm * ((N + 191) / 192) + ncu - 1) / ncu;
  return r192 * 85 < r256 * 100;
}

// The rows of a short last 256-row tile, when leaving them to the small-tile
// kernel (a second launch right after) saves the persistent kernel a round of
// tiles: a 256-row tile costs the same however few of its rows are real, while
// the small tiles (64 x 128) of the leftover rows take a fraction of a round.
// E.g. M = 54560 = 213 * 256 + 32 and N = 3072: 2568 tiles = 11 rounds of 256
// CUs, of which the last holds 8 tiles; 2556 tiles = 10 rounds plus the 32 rows
// (Wan2.2-5B ffn-down 3.89 -> 3.56 ms, N = K = 3072 -8%, qkv -3%).  Every row is
// computed the same way by either kernel, so the split changes no result.
int l4_tail_rows(int M, int N, int gbn) {
  const int64_t tm = (M + 255) / 256, rem = M % 256;
  if (rem == 0 || tm < 2) return 0;
  const int64_t tn = (N + gbn - 1) / gbn, ncu = std::max(8, cu_count() / 8 * 8);
  const int64_t r_all = (tm * tn + ncu - 1) / ncu, r_main = ((tm - 1) * tn + ncu - 1) / ncu;
  return r_main < r_all ? (int)rem : 0;
}

// A paired launch (256 x 256 tiles) when its rounds of tiles cost no more than
// the larger product alone (its own tile width) plus 0.4 of a round for the
// smaller one's separate launch (measured: 666 rows at N = 1536, K = 1536 and
// 6144 take 30-50 us beside 52-134 us rounds).  SD3.5's gated-residual
// projections, 8192 image + 666 text rows at N = 1536: 192 + 18 tiles are one
// round, against one 192-wide round plus a text launch.  qkv (N = 4608) and the
// feed-forward input (N = 6144) do not pair: the text tiles would add a round.
bool pair_pays(int M0, int M1, int N) {
  const int64_t ncu = std::max(8, cu_count() / 8 * 8), tn = (N + 255) / 256;
  const int64_t big = std::max(M0, M1), t_all = ((int64_t)(M0 + 255) / 256 + (M1 + 255) / 256) * tn;
  const int64_t tb = (big + 255) / 256;
  const int64_t r_pair = (t_all + ncu - 1) / ncu, r256 = (tb * tn + ncu - 1) / ncu,
                r192 = (tb * ((N + 191) / 192) + ncu - 1) / ncu;
  return r_pair * 100 <= std::min(r256 * 100, r192 * 85) + 40;
}

template <int EPI, int BK, int T>
int launch_tile(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias, void* C,
                int64_t ldc, int M, int N, int K, const void* R, int64_t ldr, const float* gate,
                int64_t gate_stride, const int32_t* cu, int nseg, hipStream_t stream, int row_base = 0) {
  using S = Stages<BK, T>;
  const int tiles_m = (M + S::GBM - 1) / S::GBM, tiles_n = (N + S::GBN - 1) / S::GBN;
  const int64_t tiles = (int64_t)tiles_m * tiles_n;
  const int64_t nblocks = (tiles + 7) / 8 * 8;
  DITK_REQUIRE(nblocks < (1ll << 31), "ditk_gemm: grid too large");
  gemm_kernel<EPI, BK, T><<<(unsigned)nblocks, S::GW * 64, 0, stream>>>(
      (const bf16_t*)A, lda, (const bf16_t*)W, ldw, bias, C, ldc, M, N, K, (const bf16_t*)R, ldr, gate,
      gate_stride, cu, nseg, tiles_m, tiles_n, gemm_group_m(K, tiles_n), row_base);
  return ditk_check_launch("ditk_gemm");
}

// Small tiles when the large ones would number fewer than kSmallBelow: the
// choice cannot change a result, only how many CUs take part.  Measured per CU,
// a small workgroup alone on a CU runs at about half a large one's rate and two
// sharing one at about a quarter each, so small tiles (8 per large tile) win
// while they fit about two per CU: 666-row text GEMMs 1.3-3x faster (54-72
// large tiles), 8192 x 1536 1.25-1.5x slower (192 large tiles).
constexpr int64_t kSmallBelow = 128;
template <int EPI, int BK>
int launch(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias, void* C,
           int64_t ldc, int M, int N, int K, const void* R, int64_t ldr, const float* gate,
           int64_t gate_stride, const int32_t* cu, int nseg, hipStream_t stream) {
  using L = Tile<TILE_LARGE>;
  const int64_t large_tiles = (int64_t)((M + L::GBM - 1) / L::GBM) * ((N + L::GBN - 1) / L::GBN);
  if (large_tiles < kSmallBelow)
    return launch_tile<EPI, BK, TILE_SMALL>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu, nseg, stream);
  // the large-tile kernel's epilogue addresses a wave tile's rows by 32-bit offsets
  const bool l4_strides = ldc < (1 << 22) && ldr < (1 << 22);
  const int fi = EPI == EPI_F32 || !l4_strides ? 0
                 : K % 64 == 0 && use_w192(M, N) ? 6
                 : use_l4(N, K, EPI)             ? 8
                                                 : 0;
  if (fi == 0)
    return launch_tile<EPI, BK, TILE_LARGE>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu, nseg, stream);
  const int tail = l4_tail_rows(M, N, fi * 32);
  const int Mm = M - tail;
  const int rc = fi == 6 ? launch_l4<EPI, 6>(A, lda, W, ldw, bias, C, ldc, Mm, N, K, R, ldr, gate, gate_stride, cu, nseg, stream)
                         : launch_l4<EPI, 8>(A, lda, W, ldw, bias, C, ldc, Mm, N, K, R, ldr, gate, gate_stride, cu, nseg, stream);
  if (rc != 0 || tail == 0) return rc;
  return launch_tile<EPI, BK, TILE_SMALL>(static_cast<const bf16_t*>(A) + (int64_t)Mm * lda, lda, W, ldw, bias,
                                          static_cast<bf16_t*>(C) + (int64_t)Mm * ldc, ldc, tail, N, K,
                                          R ? static_cast<const bf16_t*>(R) + (int64_t)Mm * ldr : nullptr, ldr, gate,
                                          gate_stride, cu, nseg, stream, Mm);
}

template <int EPI>
int launch_k(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias, void* C,
             int64_t ldc, int M, int N, int K, const void* R, int64_t ldr, const float* gate,
             int64_t gate_stride, const int32_t* cu, int nseg, hipStream_t stream) {
  // 64-k stages when K allows (half the barriers); the MFMA k order is the
  // same for both, so results do not depend on the choice
  return K % 64 == 0 ? launch<EPI, 64>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu, nseg, stream)
                     : launch<EPI, 32>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu, nseg, stream);
}

}  // namespace

namespace {
int gemm_validate(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias, void* C, int64_t ldc,
                  int M, int N, int K, int epilogue, const void* R, int64_t ldr, const float* gate,
                  int64_t gate_stride, const int32_t* cu_seqlens, int nseg) {
  // A, C and R may be NULL when there are no rows (an empty tensor's pointer)
  DITK_REQUIRE(W && (M == 0 || (A && C)), "ditk_gemm: null operand");
  DITK_REQUIRE(M >= 0 && N > 0 && K > 0, "ditk_gemm: bad shape M=%d N=%d K=%d", M, N, K);
  DITK_REQUIRE(K % 32 == 0, "ditk_gemm: K=%d must be a multiple of 32", K);
  DITK_REQUIRE(N % 8 == 0, "ditk_gemm: N=%d must be a multiple of 8", N);
  DITK_REQUIRE(lda % 8 == 0 && ldw % 8 == 0 && lda >= K && ldw >= K,
               "ditk_gemm: lda/ldw must be multiples of 8 and >= K");
  DITK_REQUIRE((int64_t)256 * lda < (1ll << 31) && (int64_t)256 * ldw < (1ll << 31),
               "ditk_gemm: leading dimensions too large");
  DITK_REQUIRE(((uintptr_t)A % 16) == 0 && ((uintptr_t)W % 16) == 0 && ((uintptr_t)C % 16) == 0 &&
                   ((uintptr_t)bias % 16) == 0,
               "ditk_gemm: A, W, C and bias must be 16-byte aligned");
  DITK_REQUIRE(ldc % 8 == 0 && ldc >= N, "ditk_gemm: ldc must be a multiple of 8 and >= N");
  DITK_REQUIRE(epilogue >= 0 && epilogue <= 5, "ditk_gemm: unknown epilogue %d", epilogue);
  DITK_REQUIRE(!(epilogue == EPI_GATE_RES || epilogue == EPI_RES) ||
               ((R || M == 0) && ldr % 8 == 0 && ldr >= N && ((uintptr_t)R % 16) == 0),
               "ditk_gemm: residual epilogue needs a 16-byte aligned R with ldr %% 8 == 0");
  DITK_REQUIRE(epilogue != EPI_GATE_RES || (gate_stride % 4 == 0 && ((uintptr_t)gate % 16) == 0),
               "ditk_gemm: gate rows must be 16-byte aligned");
  DITK_REQUIRE(epilogue != EPI_GATE_RES || (gate && cu_seqlens && nseg > 0),
               "ditk_gemm: gated epilogue needs gate and cu_seqlens");
  return 0;
}

int gemm_run(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias, void* C, int64_t ldc,
             int M, int N, int K, int epilogue, const void* R, int64_t ldr, const float* gate,
             int64_t gate_stride, const int32_t* cu_seqlens, int nseg, hipStream_t stream) {
  if (M == 0) return 0;
  switch (epilogue) {
    case EPI_BIAS: return launch_k<EPI_BIAS>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu_seqlens, nseg, stream);
    case EPI_GELU: return launch_k<EPI_GELU>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu_seqlens, nseg, stream);
    case EPI_GATE_RES: return launch_k<EPI_GATE_RES>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu_seqlens, nseg, stream);
    case EPI_RES: return launch_k<EPI_RES>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu_seqlens, nseg, stream);
    case EPI_F32: return launch_k<EPI_F32>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu_seqlens, nseg, stream);
    default: return launch_k<EPI_SILU>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu_seqlens, nseg, stream);
  }
}
}  // namespace

DITK_EXPORT int ditk_gemm(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias,
                          void* C, int64_t ldc, int M, int N, int K, int epilogue, const void* R,
                          int64_t ldr, const float* gate, int64_t gate_stride,
                          const int32_t* cu_seqlens, int nseg, hipStream_t stream) {
  if (int rc = gemm_validate(A, lda, W, ldw, bias, C, ldc, M, N, K, epilogue, R, ldr, gate, gate_stride,
                             cu_seqlens, nseg))
    return rc;
  return gemm_run(A, lda, W, ldw, bias, C, ldc, M, N, K, epilogue, R, ldr, gate, gate_stride, cu_seqlens, nseg,
                  stream);
}

DITK_EXPORT int ditk_gemm_pair(const void* A0, int64_t lda0, const void* W0, int64_t ldw0, const float* bias0,
                               void* C0, int64_t ldc0, int M0, const void* R0, int64_t ldr0, const float* gate0,
                               int64_t gate_stride0, const int32_t* cu_seqlens0, int nseg0, const void* A1,
                               int64_t lda1, const void* W1, int64_t ldw1, const float* bias1, void* C1,
                               int64_t ldc1, int M1, const void* R1, int64_t ldr1, const float* gate1,
                               int64_t gate_stride1, const int32_t* cu_seqlens1, int nseg1, int N, int K,
                               int epilogue, hipStream_t stream) {
  if (int rc = gemm_validate(A0, lda0, W0, ldw0, bias0, C0, ldc0, M0, N, K, epilogue, R0, ldr0, gate0,
                             gate_stride0, cu_seqlens0, nseg0))
    return rc;
  if (int rc = gemm_validate(A1, lda1, W1, ldw1, bias1, C1, ldc1, M1, N, K, epilogue, R1, ldr1, gate1,
                             gate_stride1, cu_seqlens1, nseg1))
    return rc;
  // the large-tile kernel addresses a wave tile's output and residual rows by 32-bit offsets
  const bool strides = ldc0 < (1 << 22) && ldr0 < (1 << 22) && ldc1 < (1 << 22) && ldr1 < (1 << 22);
  if (M0 > 0 && M1 > 0 && epilogue != EPI_F32 && K % 64 == 0 && strides && pair_pays(M0, M1, N)) {
    const L4Prob p0{(const bf16_t*)A0, lda0, (const bf16_t*)W0, ldw0, bias0, C0, ldc0, (const bf16_t*)R0, ldr0,
                    gate0, gate_stride0, cu_seqlens0, nseg0, M0, 0, 0};
    const L4Prob p1{(const bf16_t*)A1, lda1, (const bf16_t*)W1, ldw1, bias1, C1, ldc1, (const bf16_t*)R1, ldr1,
                    gate1, gate_stride1, cu_seqlens1, nseg1, M1, 0, 0};
    switch (epilogue) {
      case EPI_BIAS: return launch_l4_pair<EPI_BIAS>(p0, p1, N, K, stream);
      case EPI_GELU: return launch_l4_pair<EPI_GELU>(p0, p1, N, K, stream);
      case EPI_GATE_RES: return launch_l4_pair<EPI_GATE_RES>(p0, p1, N, K, stream);
      case EPI_RES: return launch_l4_pair<EPI_RES>(p0, p1, N, K, stream);
      default: return launch_l4_pair<EPI_SILU>(p0, p1, N, K, stream);
    }
  }
  if (int rc = gemm_run(A0, lda0, W0, ldw0, bias0, C0, ldc0, M0, N, K, epilogue, R0, ldr0, gate0, gate_stride0,
                        cu_seqlens0, nseg0, stream))
    return rc;
  return gemm_run(A1, lda1, W1, ldw1, bias1, C1, ldc1, M1, N, K, epilogue, R1, ldr1, gate1, gate_stride1,
                  cu_seqlens1, nseg1, stream);
}
