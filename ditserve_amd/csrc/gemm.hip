// bf16 MFMA GEMM for the DiT projections, with fused epilogues.
//
//   C[m, n] = epilogue( sum_k A[m, k] * W[n, k] + bias[n] )
//
// A is the token-major activation [M, K]; W is an nn.Linear weight [N, K]; both
// are K-contiguous, which is what the MFMA operands want (each lane feeds 8
// consecutive k values).  The kernel computes C^T tiles: the MFMA "A" operand
// is a 32-row slice of W and the "B" operand a 32-token slice of the
// activation, so every lane ends up owning one token and 4 consecutive output
// features per accumulator group -> 8-byte row-major stores.
//
// Tiling (gfx950, v_mfma_f32_32x32x16_bf16): a 512-thread workgroup computes a
// 256 (tokens) x 256 (features) tile as 2 x 4 waves of 128 tokens x 64
// features (8 accumulator tiles per wave), two waves per SIMD so one wave's
// MFMAs issue while the other waits to issue its DMA.  K advances through
// 128 KiB of LDS stages filled by direct global->LDS DMA (no register
// staging): two stages of 64 k when K % 64 == 0, else four of 32 k.  The bias
// is loaded before the k loop, so the epilogue of a bias / GELU / SiLU
// projection waits on no global load.
//
// The k-loop order is fixed and there is no split-K, so every output element is
// computed the same way whatever M is and wherever its row sits: packed and
// per-request projections agree bitwise.
#include "ditk_common.h"

#ifndef GEMM_WAVES
#define GEMM_WAVES 8  // waves per workgroup (4: one per SIMD, 8: two per SIMD)
#endif
#ifndef GEMM_BIAS_EARLY
#define GEMM_BIAS_EARLY (GEMM_WAVES == 8)  // bias loaded before the k loop
#endif

namespace {

enum Epilogue : int {
  EPI_BIAS = 0,      // bf16(acc + b)
  EPI_GELU = 1,      // bf16(gelu_tanh(bf16(acc + b)))
  EPI_GATE_RES = 2,  // bf16(R + bf16(acc + b) * gate[seg, n])   (fp32 math)
  EPI_RES = 3,       // bf16(R + bf16(acc + b))
  EPI_F32 = 4,       // fp32(acc + b)
  EPI_SILU = 5,      // bf16(silu(bf16(acc + b)))
};

constexpr int GBM = 256;                     // tokens per workgroup tile
constexpr int GBN = 256;                     // features per workgroup tile
constexpr int GW = GEMM_WAVES;               // waves per workgroup: 2 x (GW/2) wave tiles
constexpr int WTM = GBM / 2;                 // tokens per wave tile
constexpr int WTN = GBN / (GW / 2);          // features per wave tile
constexpr int NI = WTN / 32, NJ = WTM / 32;  // 32x32 MFMA tiles per wave tile
constexpr int LDS_STAGE_BYTES = 128 * 1024;  // k stages (reused by the epilogue staging)

// k-stage geometry for BK k values per stage (BK = 64 when K allows, else 32)
template <int BK>
struct Stages {
  static constexpr int GBK = BK;
  static constexpr int NCH = BK / 16;                 // 16-k MFMA chunks per stage
  static constexpr int CPRW = BK / 8;                 // 16-byte chunks per LDS row
  static constexpr int RPG = 64 / CPRW;               // rows filled by one DMA instruction (1 KiB)
  static constexpr int NGRP = GBM / RPG;              // DMA instructions per operand and stage
  static constexpr int NSTAGE = LDS_STAGE_BYTES / ((GBM + GBN) * BK * 2);
  static constexpr int DPW = NGRP / GW;               // DMA instructions per operand, wave and stage
  static_assert(GBM == GBN && (BK == 32 || BK == 64) && NSTAGE >= 2 && NCH % 2 == 0, "tile configuration");
  // LDS stage layout (A and W alike): row r of BK k-values = CPRW chunks of
  // 16 B, slot(r, u) = r*CPRW + (u ^ swz(r)).  A DMA instruction fills 64
  // contiguous slots (RPG whole rows); 16 consecutive lanes reading chunk u of
  // 16 consecutive rows hit 16 distinct 16-byte bank groups.
  static __device__ __forceinline__ int swz(int r) { return CPRW == 4 ? (r >> 2) & 3 : (r >> 1) & 7; }
  // wait until at most `stages` DMA stages (2*DPW instructions each) of this wave are in flight
  static __device__ __forceinline__ void dma_wait(int stages) {
    constexpr int P = 2 * DPW;
    if (stages >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * P) : "memory");
    else if (stages == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(P) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
};

constexpr int GROUP_M = 8;  // m-tiles per tile-order group (L2 reuse of W)

// 16 bytes per lane, global -> LDS; the wave's 64 lanes fill 1 KiB starting at
// the wave-uniform lds_slot0 (lane l writes bytes 16l .. 16l+15).
__device__ __forceinline__ void lds_dma16(const bf16_t* gsrc, u32x4_t* lds_slot0) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)gsrc,
                                   (__attribute__((address_space(3))) void*)lds_slot0, 16, 0, 0);
}
template <int EPI, int BK>
__global__ __launch_bounds__(GW * 64, 1) void gemm_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ W, int64_t ldw,
    const float* __restrict__ bias, void* __restrict__ Cv, int64_t ldc, int M, int N, int K,
    const bf16_t* R, int64_t ldr, const float* __restrict__ gate, int64_t gate_stride,
    const int32_t* __restrict__ cu, int nseg, int tiles_m, int tiles_n) {
  using S = Stages<BK>;
  constexpr int GBK = S::GBK, NCH = S::NCH, CPRW = S::CPRW, RPG = S::RPG, NSTAGE = S::NSTAGE, DPW = S::DPW;
  // 128 KiB of LDS: NSTAGE stages of A and W tiles; reused by the epilogue as
  // one [WTM tokens][WTN features] bf16 staging tile per wave.
  __shared__ u32x4_t lds[NSTAGE * (GBM + GBN) * CPRW];
  auto As = [&](int s) { return lds + s * (GBM * CPRW); };
  auto Ws = [&](int s) { return lds + NSTAGE * GBM * CPRW + s * (GBN * CPRW); };

  // XCD-aware grouped tile order: the 8 XCDs receive workgroup ids round-robin;
  // give each XCD a contiguous run of logical tiles, ordered in groups of
  // GROUP_M m-tiles so concurrently running tiles share A rows and W rows in L2.
  const int nb = gridDim.x, b = blockIdx.x;
  const int L = (b & 7) * (nb >> 3) + (b >> 3);
  if (L >= tiles_m * tiles_n) return;
  const int group = L / (GROUP_M * tiles_n);
  const int first_m = group * GROUP_M;
  const int gm = min(GROUP_M, tiles_m - first_m);
  const int pid = L % (GROUP_M * tiles_n);
  const int mt = first_m + pid % gm, nt = pid / gm;
  const int m0 = mt * GBM, n0 = nt * GBN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int wm = wave_u & 1, wn = wave_u >> 1;  // wave tile: tokens wm*WTM.., features wn*WTN..

  // ---- DMA source offsets (elements, per lane, loop invariant).  Group g of
  // 64 slots covers rows RPG*g ..; lane l -> row RPG*g + l/CPRW, stored chunk
  // l%CPRW, k chunk (l%CPRW) ^ swz(row).  Rows past M / N re-read the last row.
  const bf16_t* Ablk = A + (int64_t)m0 * lda;
  const bf16_t* Wblk = W + (int64_t)n0 * ldw;
  uint32_t a_off[DPW], w_off[DPW];  // element offsets within the workgroup's row block
#pragma unroll
  for (int i = 0; i < DPW; ++i) {
    const int g = i * GW + wave_u;
    const int row = g * RPG + lane / CPRW;
    const int ksw = ((lane % CPRW) ^ S::swz(row)) * 8;
    a_off[i] = (uint32_t)(min(row, M - 1 - m0) * lda + ksw);
    w_off[i] = (uint32_t)(min(row, N - 1 - n0) * ldw + ksw);
  }
  // DMA instruction d (0 .. 2*DPW-1) of stage kt: even d -> A, odd d -> W
  auto dma_one = [&](int kt, int d) {
    const int s = kt % NSTAGE, i = d >> 1, g = i * GW + wave_u;
    if ((d & 1) == 0) lds_dma16(Ablk + kt * GBK + a_off[i], &As(s)[g * 64]);
    else lds_dma16(Wblk + kt * GBK + w_off[i], &Ws(s)[g * 64]);
  };
  auto issue = [&](int kt) {
#pragma unroll
    for (int d = 0; d < 2 * DPW; ++d) dma_one(kt, d);
  };

  // ---- operand read bases: row 32t + l32, k chunk c*2 + hh of MFMA chunk c
  int rbase[NCH];
  {
    const int sg = S::swz(l32);
#pragma unroll
    for (int c = 0; c < NCH; ++c) rbase[c] = l32 * CPRW + ((c * 2 + hh) ^ sg);
  }
  const int a_row0 = wm * WTM, w_row0 = wn * WTN;

  // bias of the lane's accumulator features f = i*32 + gq*8 + hh*4 .. +3
  // (columns past N read the last valid group and are never stored)
  f32x4_t bvec[NI][4];
  auto load_bias = [&]() {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
        bvec[i][gq] = bias != nullptr
                          ? *reinterpret_cast<const f32x4_t*>(bias + min(n0 + w_row0 + i * 32 + gq * 8 + hh * 4, N - 4))
                          : f32x4_t{0.f, 0.f, 0.f, 0.f};
  };
  if (GEMM_BIAS_EARLY) load_bias();

  f32x16_t acc[NI][NJ];  // [feature tile i][token tile j]
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nk = K / GBK;
  auto read_chunk = [&](int s, int c, bf16x8_t (&af)[NI], bf16x8_t (&bf)[NJ]) {
#pragma unroll
    for (int i = 0; i < NI; ++i) af[i] = __builtin_bit_cast(bf16x8_t, Ws(s)[rbase[c] + (w_row0 + i * 32) * CPRW]);
#pragma unroll
    for (int j = 0; j < NJ; ++j) bf[j] = __builtin_bit_cast(bf16x8_t, As(s)[rbase[c] + (a_row0 + j * 32) * CPRW]);
  };
  // operand read r (0 .. NI+NJ-1) of chunk c from stage s into (af, bf)
  auto read_one = [&](int s, int c, int r, bf16x8_t (&af)[NI], bf16x8_t (&bf)[NJ]) {
    if (r < NI) af[r] = __builtin_bit_cast(bf16x8_t, Ws(s)[rbase[c] + (w_row0 + r * 32) * CPRW]);
    else bf[r - NI] = __builtin_bit_cast(bf16x8_t, As(s)[rbase[c] + (a_row0 + (r - NI) * 32) * CPRW]);
  };

  // Pipeline over k stages (NCH chunks of 16 k each).  Iteration kt: part A
  // runs the MFMAs of chunks 0..NCH-2 while reading chunks 1..NCH-1; then this
  // wave waits for its DMA of stage kt+1 and a barrier publishes that stage and
  // frees buffer kt (all its operand reads are in registers); part B runs chunk
  // NCH-1's MFMAs while reading chunk 0 of stage kt+1 and issuing the DMA of
  // stage kt+NSTAGE into the freed buffer.  A plain s_barrier (no release fence,
  // which would drain every stage in flight) suffices because each wave waits
  // for its own DMA with vmcnt first.  MFMAs, operand reads and DMA issues are
  // interleaved in groups fenced by sched_barrier.
#pragma unroll
  for (int kt = 0; kt < NSTAGE; ++kt)
    if (kt < nk) issue(kt);
  bf16x8_t fa[2][NI], fb[2][NJ];
  S::dma_wait(min(NSTAGE - 1, nk - 1));
  __syncthreads();
  read_chunk(0, 0, fa[0], fb[0]);

  auto publish = [&]() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
  };
  constexpr int NM = NI * NJ;  // MFMAs per chunk
  constexpr int NR = NI + NJ;  // operand reads per chunk
  constexpr int NQ = NM / 2;   // groups of 2 MFMAs per chunk
  constexpr int RPQ = (NR + NQ - 1) / NQ;           // operand reads per group
  constexpr int DPQ = (2 * DPW + NQ - 1) / NQ;      // DMA issues per group of part B
  // one interleave group: 2 MFMAs of the current chunk (operand set p), reads of chunk cn of
  // stage sn into set p^1, DMA issues d0.. of stage kd
  auto step = [&](int q, int p, int sn, int cn, int kd, bool reads, bool dmas) {
    const int x0 = 2 * q, i0 = x0 / NJ, j0 = x0 % NJ;
    acc[i0][j0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[p][i0], fb[p][j0], acc[i0][j0], 0, 0, 0);
    acc[i0][j0 + 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[p][i0], fb[p][j0 + 1], acc[i0][j0 + 1], 0, 0, 0);
    if (reads) {
#pragma unroll
      for (int r = q * RPQ; r < q * RPQ + RPQ; ++r)
        if (r < NR) read_one(sn, cn, r, fa[p ^ 1], fb[p ^ 1]);
    }
    if (dmas) {
#pragma unroll
      for (int d = q * DPQ; d < q * DPQ + DPQ; ++d)
        if (d < 2 * DPW) dma_one(kd, d);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  int kt = 0;
  // steady state: every stage has a successor and a DMA to issue
  for (; kt + NSTAGE < nk; ++kt) {
    const int s = kt % NSTAGE;
#pragma unroll
    for (int c = 0; c + 1 < NCH; ++c)
#pragma unroll
      for (int q = 0; q < NQ; ++q) step(q, c & 1, s, c + 1, 0, true, false);
    S::dma_wait(NSTAGE - 2);  // stage kt+1 landed (this wave)
    publish();
#pragma unroll
    for (int q = 0; q < NQ; ++q) step(q, 1, (kt + 1) % NSTAGE, 0, kt + NSTAGE, true, true);
  }
  // drain: no more DMA to issue
  for (; kt < nk; ++kt) {
    const int s = kt % NSTAGE;
#pragma unroll
    for (int c = 0; c + 1 < NCH; ++c)
#pragma unroll
      for (int q = 0; q < NQ; ++q) step(q, c & 1, s, c + 1, 0, true, false);
    const bool next = kt + 1 < nk;
    if (next) {
      S::dma_wait(nk - 2 - kt);
      publish();
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) step(q, 1, (kt + 1) % NSTAGE, 0, 0, next, false);
  }
  __syncthreads();

  // ---------------------------------------------------------------- epilogue
  if (!GEMM_BIAS_EARLY) load_bias();
  // Accumulator lane layout: token t = j*32 + l32 of the wave tile, features
  // f = i*32 + g*8 + hh*4 + e.
  if (EPI == EPI_F32) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int m = m0 + a_row0 + j * 32 + l32;
      if (m >= M) continue;
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int n = n0 + w_row0 + i * 32 + gq * 8 + hh * 4;
          if (n >= N) continue;
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = acc[i][j][gq * 4 + e] + bvec[i][gq][e];
          float* C = reinterpret_cast<float*>(Cv) + (int64_t)m * ldc + n;
          *reinterpret_cast<f32x4_t*>(C) = f32x4_t{o[0], o[1], o[2], o[3]};
        }
    }
    return;
  }
  // bf16 epilogues: y = bf16(acc + bias) goes through a per-wave LDS tile
  // [WTM tokens][WTN features] (16-byte chunk c of row t stored at c ^ (t % CPR)),
  // then rows are read back so residual / gate loads and output stores are
  // 16-byte coalesced.  Lane (c, row group) handles features n..n+7 of rows
  // t = r*RPP + lane/CPR; its residual rows and gate are loaded before the
  // staging, so their latency overlaps it instead of stalling each row.
  constexpr int CPR = WTN / 8;   // 16-byte chunks per staged row
  constexpr int RPP = 64 / CPR;  // rows per pass of the wave
  constexpr int NPASS = WTM / RPP;  // passes
  constexpr bool HAS_RES = EPI == EPI_GATE_RES || EPI == EPI_RES;
  const int c = lane % CPR;
  const int n = n0 + w_row0 + c * 8;
  const int mrow = m0 + a_row0 + lane / CPR;  // row of pass 0; pass r adds r*RPP
  u32x4_t res[HAS_RES ? NPASS : 1];
  if (HAS_RES) {
#pragma unroll
    for (int r = 0; r < NPASS; ++r) {
      const int m = mrow + r * RPP;
      res[r] = (m < M && n < N) ? *reinterpret_cast<const u32x4_t*>(R + (int64_t)m * ldr + n) : u32x4_t{0, 0, 0, 0};
    }
  }
  // gate rows: one segment for the whole wave tile (the common case) loads its
  // gate once; a tile that straddles a segment boundary looks it up per row
  int seg_lo = 0;
  bool one_seg = true;
  f32x4_t g0 = {0.f, 0.f, 0.f, 0.f}, g1 = {0.f, 0.f, 0.f, 0.f};
  if (EPI == EPI_GATE_RES) {
    seg_lo = find_segment(cu, nseg, m0 + a_row0);
    one_seg = seg_lo == find_segment(cu, nseg, min(m0 + a_row0 + WTM, M) - 1);
    if (one_seg && n < N) {
      const float* g = gate + (int64_t)seg_lo * gate_stride + n;
      g0 = *reinterpret_cast<const f32x4_t*>(g);
      g1 = *reinterpret_cast<const f32x4_t*>(g + 4);
    }
  }
  u32x2_t* stage8 = reinterpret_cast<u32x2_t*>(lds + wave_u * (WTM * CPR));
  const u32x4_t* stage16 = lds + wave_u * (WTM * CPR);
  static_assert(NSTAGE * (GBM + GBN) * CPRW >= GW * WTM * CPR, "epilogue staging exceeds the LDS stages");
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const f32x4_t b4 = bvec[i][gq];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int t = j * 32 + l32;
        const int chunk = (i * 4 + gq) ^ (t % CPR);
        stage8[(t * CPR + chunk) * 2 + hh] =
            u32x2_t{pack_bf2(acc[i][j][gq * 4 + 0] + b4[0], acc[i][j][gq * 4 + 1] + b4[1]),
                    pack_bf2(acc[i][j][gq * 4 + 2] + b4[2], acc[i][j][gq * 4 + 3] + b4[3])};
      }
    }
  __syncthreads();
  if (n >= N) return;
#pragma unroll
  for (int r = 0; r < NPASS; ++r) {
    const int t = r * RPP + lane / CPR;
    const int m = mrow + r * RPP;
    if (m >= M) continue;
    u32x4_t v = stage16[t * CPR + (c ^ (t % CPR))];
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
            const float* g = gate + (int64_t)find_segment(cu, nseg, m) * gate_stride + n;
            h0 = *reinterpret_cast<const f32x4_t*>(g);
            h1 = *reinterpret_cast<const f32x4_t*>(g + 4);
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
    *reinterpret_cast<u32x4_t*>(reinterpret_cast<bf16_t*>(Cv) + (int64_t)m * ldc + n) = v;
  }
}

template <int EPI, int BK>
int launch(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias, void* C,
           int64_t ldc, int M, int N, int K, const void* R, int64_t ldr, const float* gate,
           int64_t gate_stride, const int32_t* cu, int nseg, hipStream_t stream) {
  const int tiles_m = (M + GBM - 1) / GBM, tiles_n = (N + GBN - 1) / GBN;
  const int64_t tiles = (int64_t)tiles_m * tiles_n;
  const int64_t nblocks = (tiles + 7) / 8 * 8;
  DITK_REQUIRE(nblocks < (1ll << 31), "ditk_gemm: grid too large");
  gemm_kernel<EPI, BK><<<(unsigned)nblocks, GW * 64, 0, stream>>>(
      (const bf16_t*)A, lda, (const bf16_t*)W, ldw, bias, C, ldc, M, N, K, (const bf16_t*)R, ldr, gate,
      gate_stride, cu, nseg, tiles_m, tiles_n);
  return ditk_check_launch("ditk_gemm");
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

DITK_EXPORT int ditk_gemm(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias,
                          void* C, int64_t ldc, int M, int N, int K, int epilogue, const void* R,
                          int64_t ldr, const float* gate, int64_t gate_stride,
                          const int32_t* cu_seqlens, int nseg, hipStream_t stream) {
  DITK_REQUIRE(A && W && C, "ditk_gemm: null operand");
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
               (R && ldr % 8 == 0 && ldr >= N && ((uintptr_t)R % 16) == 0),
               "ditk_gemm: residual epilogue needs a 16-byte aligned R with ldr %% 8 == 0");
  DITK_REQUIRE(epilogue != EPI_GATE_RES || (gate_stride % 4 == 0 && ((uintptr_t)gate % 16) == 0),
               "ditk_gemm: gate rows must be 16-byte aligned");
  DITK_REQUIRE(epilogue != EPI_GATE_RES || (gate && cu_seqlens && nseg > 0),
               "ditk_gemm: gated epilogue needs gate and cu_seqlens");
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
