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
// Tiling (gfx950, v_mfma_f32_32x32x16_bf16): a 256-thread workgroup computes a
// WG_M (tokens) x WG_N (features) tile with 2x2 waves; K advances in steps of
// 32 through double-buffered LDS (XOR-swizzled 16-byte chunks, conflict-free
// for the 32-row operand reads) with the next step's global loads held in
// registers while the current step's MFMAs run.
//
// The k-loop order is fixed and there is no split-K, so every output element is
// computed the same way whatever M is and wherever its row sits: packed and
// per-request projections agree bitwise.
#include "ditk_common.h"

namespace {

enum Epilogue : int {
  EPI_BIAS = 0,      // bf16(acc + b)
  EPI_GELU = 1,      // bf16(gelu_tanh(bf16(acc + b)))
  EPI_GATE_RES = 2,  // bf16(R + bf16(acc + b) * gate[seg, n])   (fp32 math)
  EPI_RES = 3,       // bf16(R + bf16(acc + b))
  EPI_F32 = 4,       // fp32(acc + b)
  EPI_SILU = 5,      // bf16(silu(bf16(acc + b)))
};

constexpr int BK = 32;  // k elements per LDS stage (4 x 16-byte chunks per row)

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 2) & 3); }

template <int EPI, int WG_M, int WG_N>
__global__ __launch_bounds__(256, 1) void gemm_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ W, int64_t ldw,
    const float* __restrict__ bias, void* __restrict__ Cv, int64_t ldc, int M, int N, int K,
    const bf16_t* R, int64_t ldr, const float* __restrict__ gate, int64_t gate_stride,
    const int32_t* __restrict__ cu, int nseg, int tiles_n) {
  constexpr int TJ = WG_M / 64;  // token MFMA tiles per wave
  constexpr int TI = WG_N / 64;  // feature MFMA tiles per wave
  constexpr int A_LOADS = WG_M * 4 / 256;
  constexpr int W_LOADS = WG_N * 4 / 256;
  __shared__ u32x4_t As[2][WG_M * 4];
  __shared__ u32x4_t Ws[2][WG_N * 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int l32 = lane & 31, h = lane >> 5;

  const int tile = blockIdx.x;
  const int mt = tile / tiles_n, nt = tile % tiles_n;
  const int m0 = mt * WG_M, n0 = nt * WG_N;

  // global -> register staging
  const int ld_row = tid >> 2, ld_chunk = tid & 3;
  u32x4_t ra[A_LOADS], rw[W_LOADS];
  const int nk = (K + BK - 1) / BK;

  auto gload = [&](int kt) {
    const int k = kt * BK + ld_chunk * 8;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      int r = m0 + ld_row + i * 64;
      if (r < M && k < K) ra[i] = *reinterpret_cast<const u32x4_t*>(A + (int64_t)r * lda + k);
      else ra[i] = u32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < W_LOADS; ++i) {
      int r = n0 + ld_row + i * 64;
      if (r < N && k < K) rw[i] = *reinterpret_cast<const u32x4_t*>(W + (int64_t)r * ldw + k);
      else rw[i] = u32x4_t{0, 0, 0, 0};
    }
  };
  auto lstore = [&](int s) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      int r = ld_row + i * 64;
      As[s][r * 4 + swz(r, ld_chunk)] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < W_LOADS; ++i) {
      int r = ld_row + i * 64;
      Ws[s][r * 4 + swz(r, ld_chunk)] = rw[i];
    }
  };

  f32x16_t acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  gload(0);
  lstore(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int s = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const int chunk = kc * 2 + h;
      bf16x8_t af[TI], bfr[TJ];
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        int r = wn * (WG_N / 2) + i * 32 + l32;
        af[i] = __builtin_bit_cast(bf16x8_t, Ws[s][r * 4 + swz(r, chunk)]);
      }
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        int r = wm * (WG_M / 2) + j * 32 + l32;
        bfr[j] = __builtin_bit_cast(bf16x8_t, As[s][r * 4 + swz(r, chunk)]);
      }
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) lstore(s ^ 1);
    __syncthreads();
  }

  // ---------------------------------------------------------------- epilogue
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int m = m0 + wm * (WG_M / 2) + j * 32 + l32;
    if (m >= M) continue;
    const float* g = nullptr;
    if (EPI == EPI_GATE_RES) g = gate + (int64_t)find_segment(cu, nseg, m) * gate_stride;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int n = n0 + wn * (WG_N / 2) + i * 32 + gq * 8 + h * 4;
        if (n >= N) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = acc[i][j][gq * 4 + e];
          if (bias != nullptr) t += bias[n + e];
          o[e] = t;
        }
        if (EPI == EPI_F32) {
          float* C = reinterpret_cast<float*>(Cv) + (int64_t)m * ldc + n;
          *reinterpret_cast<f32x4_t*>(C) = f32x4_t{o[0], o[1], o[2], o[3]};
          continue;
        }
        if (EPI != EPI_BIAS) {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = round_bf(o[e]);
        }
        if (EPI == EPI_GELU) {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = gelu_tanh_f(o[e]);
        } else if (EPI == EPI_SILU) {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = silu_f(o[e]);
        } else if (EPI == EPI_GATE_RES || EPI == EPI_RES) {
          u32x2_t rr = *reinterpret_cast<const u32x2_t*>(R + (int64_t)m * ldr + n);
          float rv[4] = {__uint_as_float(rr[0] << 16), __uint_as_float(rr[0] & 0xffff0000u),
                         __uint_as_float(rr[1] << 16), __uint_as_float(rr[1] & 0xffff0000u)};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o[e] = (EPI == EPI_GATE_RES) ? fmaf(o[e], g[n + e], rv[e]) : (rv[e] + o[e]);
        }
        bf16_t* C = reinterpret_cast<bf16_t*>(Cv) + (int64_t)m * ldc + n;
        *reinterpret_cast<u32x2_t*>(C) = u32x2_t{pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3])};
      }
    }
  }
}

template <int EPI>
int launch(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias, void* C,
           int64_t ldc, int M, int N, int K, const void* R, int64_t ldr, const float* gate,
           int64_t gate_stride, const int32_t* cu, int nseg, hipStream_t stream) {
  constexpr int WG_M = 256, WG_N = 128;
  int tiles_m = (M + WG_M - 1) / WG_M, tiles_n = (N + WG_N - 1) / WG_N;
  gemm_kernel<EPI, WG_M, WG_N><<<tiles_m * tiles_n, 256, 0, stream>>>(
      (const bf16_t*)A, lda, (const bf16_t*)W, ldw, bias, C, ldc, M, N, K, (const bf16_t*)R, ldr, gate,
      gate_stride, cu, nseg, tiles_n);
  return ditk_check_launch("ditk_gemm");
}

}  // namespace

DITK_EXPORT int ditk_gemm(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias,
                          void* C, int64_t ldc, int M, int N, int K, int epilogue, const void* R,
                          int64_t ldr, const float* gate, int64_t gate_stride,
                          const int32_t* cu_seqlens, int nseg, hipStream_t stream) {
  DITK_REQUIRE(A && W && C, "ditk_gemm: null operand");
  DITK_REQUIRE(M >= 0 && N > 0 && K > 0, "ditk_gemm: bad shape M=%d N=%d K=%d", M, N, K);
  DITK_REQUIRE(K % 8 == 0, "ditk_gemm: K=%d must be a multiple of 8", K);
  DITK_REQUIRE(N % 4 == 0, "ditk_gemm: N=%d must be a multiple of 4", N);
  DITK_REQUIRE(lda % 8 == 0 && ldw % 8 == 0 && lda >= K && ldw >= K,
               "ditk_gemm: lda/ldw must be multiples of 8 and >= K");
  DITK_REQUIRE(ldc % 4 == 0 && ldc >= N, "ditk_gemm: ldc must be a multiple of 4 and >= N");
  DITK_REQUIRE(epilogue >= 0 && epilogue <= 5, "ditk_gemm: unknown epilogue %d", epilogue);
  DITK_REQUIRE(!(epilogue == EPI_GATE_RES || epilogue == EPI_RES) || (R && ldr % 4 == 0 && ldr >= N),
               "ditk_gemm: residual epilogue needs R with ldr %% 4 == 0");
  DITK_REQUIRE(epilogue != EPI_GATE_RES || (gate && cu_seqlens && nseg > 0),
               "ditk_gemm: gated epilogue needs gate and cu_seqlens");
  if (M == 0) return 0;
  switch (epilogue) {
    case EPI_BIAS: return launch<EPI_BIAS>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu_seqlens, nseg, stream);
    case EPI_GELU: return launch<EPI_GELU>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu_seqlens, nseg, stream);
    case EPI_GATE_RES: return launch<EPI_GATE_RES>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu_seqlens, nseg, stream);
    case EPI_RES: return launch<EPI_RES>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu_seqlens, nseg, stream);
    case EPI_F32: return launch<EPI_F32>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu_seqlens, nseg, stream);
    default: return launch<EPI_SILU>(A, lda, W, ldw, bias, C, ldc, M, N, K, R, ldr, gate, gate_stride, cu_seqlens, nseg, stream);
  }
}
