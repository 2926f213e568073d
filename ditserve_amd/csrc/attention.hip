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
// Per workgroup: 4 waves x 64 queries of one (segment, head); K/Vt tiles of 64
// keys are staged through double-buffered LDS.  Each wave computes
//   S^T = K Q^T        (A = K rows from LDS, B = Q held in registers)
//   P^T = exp2(S^T * scale*log2e - m)   (online softmax, fp32)
//   O^T += Vt P^T      (A = Vt rows from LDS, B = P^T straight from registers)
// with v_mfma_f32_32x32x16_bf16.  The K rows fed to the first MFMA are permuted
// (kperm) so that the S^T accumulator registers of each lane are exactly the
// B-operand layout of the second MFMA: no shuffles between the two products.
// Each lane owns one query of each 32-query tile, so softmax statistics are
// per-lane scalars combined across the two half-waves with one shuffle.
//
// Query tiles start at each segment's first query and the key loop starts at
// each segment's first key, so results are independent of packing: a request
// packed with others is bitwise equal to the same request run alone.
#include "ditk_common.h"

namespace {

constexpr int BM = 256;  // queries per workgroup (4 waves x 64)
constexpr int BN = 64;   // keys per iteration

// S^T row m of a 32-key MFMA tile holds key kperm(m): with the D layout
// row = (v/4)*8 + (lane/32)*4 + v%4, this puts key (v/8)*16 + (lane/32)*8 + v%8
// in accumulator register v — the B-operand k-slot order of the PV product.
__device__ __forceinline__ int kperm(int m) {
  return ((m >> 4) << 4) | (((m >> 2) & 1) << 3) | (((m >> 3) & 1) << 2) | (m & 3);
}

template <int HD>
__device__ __forceinline__ int k_swz(int row, int chunk) {
  if (HD == 128) return chunk ^ (row & 15);
  return chunk ^ ((row >> 1) & 7);
}
__device__ __forceinline__ int v_swz(int d, int chunk) { return chunk ^ ((d >> 1) & 7); }

// 16 bytes per lane, global -> LDS; the 64 lanes of the wave fill 1 KiB of LDS
// starting at the wave-uniform `lds_slot0` (lane l writes bytes l*16..l*16+15).
__device__ __forceinline__ void lds_dma16(const bf16_t* gsrc, u32x4_t* lds_slot0) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)gsrc,
                                   (__attribute__((address_space(3))) void*)lds_slot0, 16, 0, 0);
}

__device__ __forceinline__ void dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

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

template <int HD>
__global__ __launch_bounds__(256, 1) void flash_fwd_kernel(
    const bf16_t* __restrict__ Q, int64_t ldq, const bf16_t* __restrict__ Kp, int64_t ldk,
    const bf16_t* __restrict__ Vt, int64_t vt_ld, int64_t vt_hs, bf16_t* __restrict__ O, int64_t ldo,
    float* __restrict__ lse, int64_t lse_ld, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ cu_k, int nseg, int heads, int tiles_bound, float scale_log2) {
  constexpr int NC = HD / 16;       // 16-wide k chunks of the head dim
  constexpr int KCH = HD / 8;       // 16-byte chunks per K row
  constexpr int K_LOADS = BN * KCH / 256;
  constexpr int V_LOADS = HD * (BN / 8) / 256;
  constexpr int DT = HD / 32;       // 32-row d tiles of O^T
  __shared__ u32x4_t Ks[2][BN * KCH];
  __shared__ u32x4_t Vs[2][HD * (BN / 8)];

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
  const int q_end = cu_q[seg + 1];
  const int qbase = cu_q[seg] + t * BM + wave * 64;
  const int k_beg = cu_k[seg], k_len = cu_k[seg + 1] - k_beg;
  const int pk = padded_key_start(cu_k, seg);

  const bf16_t* Qh = Q + (int64_t)head * HD;
  const bf16_t* Kh = Kp + (int64_t)head * HD;
  const bf16_t* Vh = Vt + (int64_t)head * vt_hs + pk;

  // ---- Q fragments (B operand of S^T): lane -> query l32, k-slot hh*8..+8
  bf16x8_t qf[2][NC];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    int row = qbase + qt * 32 + l32;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      u32x4_t v = u32x4_t{0, 0, 0, 0};
      if (row < q_end) v = *reinterpret_cast<const u32x4_t*>(Qh + (int64_t)row * ldq + c * 16 + hh * 8);
      qf[qt][c] = __builtin_bit_cast(bf16x8_t, v);
    }
  }

  f32x16_t o[DT][2];
#pragma unroll
  for (int d = 0; d < DT; ++d)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[d][qt][v] = 0.f;
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.f, 0.f};

  // ---- tile staging: direct global -> LDS 16-byte DMA (no register staging).
  // Lane l of load instruction i of wave w fills LDS chunk slot
  // P = (i*4 + w)*64 + l; the XOR swizzle is applied by choosing which global
  // chunk lands in that slot.  K rows past the segment end read the segment's
  // last row (finite data; those keys are masked to -inf), Vt padding is zero.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  auto issue = [&](int kt, int s) {
    const int kb = kt * BN;
#pragma unroll
    for (int i = 0; i < K_LOADS; ++i) {
      const int slot0 = (i * 4 + wave_u) * 64;
      const int P = slot0 + lane;
      const int r = P / KCH, ch = k_swz<HD>(r, P % KCH);
      const int kr = min(kb + r, k_len - 1);
      lds_dma16(Kh + (int64_t)(k_beg + kr) * ldk + ch * 8, &Ks[s][slot0]);
    }
#pragma unroll
    for (int i = 0; i < V_LOADS; ++i) {
      const int slot0 = (i * 4 + wave_u) * 64;
      const int P = slot0 + lane;
      const int d = P >> 3, ch = v_swz(d, P & 7);
      lds_dma16(Vh + (int64_t)d * vt_ld + kb + ch * 8, &Vs[s][slot0]);
    }
  };

  const int nkt = (k_len + BN - 1) / BN;
  if (nkt > 0) issue(0, 0);
  dma_wait();
  __syncthreads();

  for (int kt = 0; kt < nkt; ++kt) {
    const int s = kt & 1;
    if (kt + 1 < nkt) issue(kt + 1, s ^ 1);

    // ---- S^T = K Q^T  (2 key tiles x 2 query tiles)
    f32x16_t sacc[2][2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int v = 0; v < 16; ++v) sacc[kk][qt][v] = 0.f;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int r = kk * 32 + kperm(l32);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        bf16x8_t kf = __builtin_bit_cast(bf16x8_t, Ks[s][r * KCH + k_swz<HD>(r, c * 2 + hh)]);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
          sacc[kk][qt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[qt][c], sacc[kk][qt], 0, 0, 0);
      }
    }

    // ---- online softmax (per lane: one query per query tile)
    const int valid = k_len - kt * BN;  // keys of this tile that exist
    uint32_t pf[2][2][2][4];            // [qt][kk][j] 8 bf16 each
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float mx = -INFINITY;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          int key = kk * 32 + (v >> 3) * 16 + hh * 8 + (v & 7);
          float x = sacc[kk][qt][v];
          if (valid < BN && key >= valid) x = -INFINITY;
          sacc[kk][qt][v] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run[qt], mx * scale_log2);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = exp2f(m_run[qt] - m_use);
      m_run[qt] = m_new;
      float rs = 0.f;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float p0 = exp2f(fmaf(sacc[kk][qt][j * 8 + 2 * e], scale_log2, -m_use));
            float p1 = exp2f(fmaf(sacc[kk][qt][j * 8 + 2 * e + 1], scale_log2, -m_use));
            rs += p0 + p1;
            pf[qt][kk][j][e] = pack_bf2(p0, p1);
          }
      l_run[qt] = l_run[qt] * alpha + rs;
      if (alpha != 1.f) {
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
          for (int v = 0; v < 16; ++v) o[d][qt][v] *= alpha;
      }
    }

    // ---- O^T += Vt P^T
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const int dr = d * 32 + l32;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          bf16x8_t vf = __builtin_bit_cast(bf16x8_t, Vs[s][dr * 8 + v_swz(dr, kk * 4 + j * 2 + hh)]);
#pragma unroll
          for (int qt = 0; qt < 2; ++qt) {
            u32x4_t pv = u32x4_t{pf[qt][kk][j][0], pf[qt][kk][j][1], pf[qt][kk][j][2], pf[qt][kk][j][3]};
            o[d][qt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, __builtin_bit_cast(bf16x8_t, pv), o[d][qt], 0, 0, 0);
          }
        }
    }

    dma_wait();
    __syncthreads();
  }

  // ---- normalise and store
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float l = l_run[qt] + __shfl_xor(l_run[qt], 32, 64);
    const int row = qbase + qt * 32 + l32;
    if (row >= q_end) continue;
    const float inv = (l > 0.f) ? 1.f / l : 0.f;
    bf16_t* orow = O + (int64_t)row * ldo + (int64_t)head * HD;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dd = d * 32 + g * 8 + hh * 4;
        u32x2_t w = u32x2_t{pack_bf2(o[d][qt][g * 4 + 0] * inv, o[d][qt][g * 4 + 1] * inv),
                            pack_bf2(o[d][qt][g * 4 + 2] * inv, o[d][qt][g * 4 + 3] * inv)};
        *reinterpret_cast<u32x2_t*>(orow + dd) = w;
      }
    if (lse != nullptr && hh == 0)
      lse[(int64_t)head * lse_ld + row] =
          (l > 0.f) ? (m_run[qt] + log2f(l)) * 0.6931471805599453f : -INFINITY;
  }
}

// V [Tk, ldv] (head h at columns h*HD..) -> Vt [heads][HD][vt_ld], per-segment
// 64-aligned columns, zero padding.  One workgroup per (64-key tile, head).
template <int HD>
__global__ __launch_bounds__(256) void transpose_v_kernel(const bf16_t* __restrict__ V, int64_t ldv,
                                                          bf16_t* __restrict__ Vt, int64_t vt_ld,
                                                          int64_t vt_hs, const int32_t* __restrict__ cu,
                                                          int nseg) {
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
    if (k0 + r < k_end) v = *reinterpret_cast<const u32x4_t*>(Vh + (int64_t)(k0 + r) * ldv + ch * 8);
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

DITK_EXPORT int ditk_transpose_v(const void* v, int64_t ldv, void* vt, int64_t vt_ld, int Tk,
                                 int heads, int head_dim, const int32_t* cu_k, int nseg,
                                 hipStream_t stream) {
  DITK_REQUIRE(v && vt && cu_k, "ditk_transpose_v: null tensor");
  DITK_REQUIRE(head_dim == 64 || head_dim == 128, "ditk_transpose_v: head_dim must be 64 or 128");
  DITK_REQUIRE(nseg > 0 && heads > 0 && Tk >= 0, "ditk_transpose_v: bad sizes");
  DITK_REQUIRE(ldv % 8 == 0 && vt_ld % 8 == 0, "ditk_transpose_v: leading dims must be multiples of 8");
  DITK_REQUIRE(vt_ld >= ditk_vt_columns(Tk, nseg), "ditk_transpose_v: vt_ld=%lld < required %lld",
               (long long)vt_ld, (long long)ditk_vt_columns(Tk, nseg));
  DITK_REQUIRE(((uintptr_t)v % 16) == 0 && ((uintptr_t)vt % 16) == 0, "ditk_transpose_v: misaligned");
  if (Tk == 0) return 0;
  dim3 grid((unsigned)((Tk + BN - 1) / BN + nseg), (unsigned)heads);
  const int64_t hs = (int64_t)head_dim * vt_ld;
  if (head_dim == 128)
    transpose_v_kernel<128><<<grid, 256, 0, stream>>>((const bf16_t*)v, ldv, (bf16_t*)vt, vt_ld, hs, cu_k, nseg);
  else
    transpose_v_kernel<64><<<grid, 256, 0, stream>>>((const bf16_t*)v, ldv, (bf16_t*)vt, vt_ld, hs, cu_k, nseg);
  return ditk_check_launch("ditk_transpose_v");
}

DITK_EXPORT int ditk_flash_attn_varlen(const void* q, int64_t ldq, const void* k, int64_t ldk,
                                       const void* vt, int64_t vt_ld, void* o, int64_t ldo,
                                       float* lse, int64_t lse_ld, const int32_t* cu_q,
                                       const int32_t* cu_k, int nseg, int Tq, int heads,
                                       int head_dim, float softmax_scale, hipStream_t stream) {
  DITK_REQUIRE(q && k && vt && o && cu_q && cu_k, "ditk_flash_attn_varlen: null tensor");
  DITK_REQUIRE(head_dim == 64 || head_dim == 128, "ditk_flash_attn_varlen: head_dim must be 64 or 128, got %d", head_dim);
  DITK_REQUIRE(nseg > 0 && heads > 0 && Tq >= 0, "ditk_flash_attn_varlen: bad sizes");
  DITK_REQUIRE(ldq % 8 == 0 && ldk % 8 == 0 && ldo % 4 == 0 && vt_ld % 8 == 0,
               "ditk_flash_attn_varlen: leading dims must be multiples of 8 (ldo of 4)");
  DITK_REQUIRE(((uintptr_t)q % 16) == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)vt % 16) == 0 &&
               ((uintptr_t)o % 8) == 0, "ditk_flash_attn_varlen: misaligned tensor");
  DITK_REQUIRE(softmax_scale > 0.f, "ditk_flash_attn_varlen: softmax_scale must be > 0");
  if (Tq == 0) return 0;
  const int tiles_bound = (Tq + BM - 1) / BM + nseg;
  int64_t nblocks = (int64_t)tiles_bound * heads;
  nblocks = (nblocks + 7) / 8 * 8;
  DITK_REQUIRE(nblocks < (1ll << 31), "ditk_flash_attn_varlen: grid too large");
  const float sl2 = softmax_scale * 1.4426950408889634f;
  const int64_t hs = (int64_t)head_dim * vt_ld;
  if (head_dim == 128)
    flash_fwd_kernel<128><<<(unsigned)nblocks, 256, 0, stream>>>(
        (const bf16_t*)q, ldq, (const bf16_t*)k, ldk, (const bf16_t*)vt, vt_ld, hs, (bf16_t*)o, ldo, lse,
        lse_ld, cu_q, cu_k, nseg, heads, tiles_bound, sl2);
  else
    flash_fwd_kernel<64><<<(unsigned)nblocks, 256, 0, stream>>>(
        (const bf16_t*)q, ldq, (const bf16_t*)k, ldk, (const bf16_t*)vt, vt_ld, hs, (bf16_t*)o, ldo, lse,
        lse_ld, cu_q, cu_k, nseg, heads, tiles_bound, sl2);
  return ditk_check_launch("ditk_flash_attn_varlen");
}
