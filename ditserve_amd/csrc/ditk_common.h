// Shared helpers for the ditk HIP kernels (gfx950 / CDNA4 only).
//
// Conventions used by every kernel in this library:
//   * activations and weights are bf16 stored as uint16_t, row-major, with an
//     explicit leading dimension (elements) per tensor;
//   * accumulation and all normalisation / modulation math is fp32;
//   * float -> bf16 is round-to-nearest-even (NaN stays NaN);
//   * packed batches are described by an int32 cu_seqlens table on the device;
//     a token's segment is found by binary search, so per-token results never
//     depend on where a segment sits in the packed buffer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define DITK_EXPORT extern "C" __attribute__((visibility("default")))

typedef uint16_t bf16_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2_t;

// ---------------------------------------------------------------------------
// error plumbing (host)
// ---------------------------------------------------------------------------
void ditk_set_error(const char* fmt, ...);
int ditk_check_launch(const char* what);

// Jobs of the multi-job row-kernel entry points; the same layout as the
// declarations of include/ditk.h (C ABI).
struct ditk_adaln_job {
  const void* x;
  int64_t ldx;
  void* y;
  int64_t ldy;
  const int32_t* cu_seqlens;
  const float* shift;
  const float* scale;
  int64_t mod_stride;
  const float* weight;
  const float* bias;
  int T, D, nseg, norm_kind;
  float eps;
};
static_assert(sizeof(ditk_adaln_job) == 104, "ditk_adaln_job layout");

struct ditk_qk_norm_job {
  const void* q;
  int64_t ldq;
  const void* k;
  int64_t ldk;
  void* q_out;
  int64_t ldqo;
  void* k_out;
  int64_t ldko;
  const float* wq;
  const float* wk;
  int T, D, head_dim, per_head;
  float eps;
};
static_assert(sizeof(ditk_qk_norm_job) == 104, "ditk_qk_norm_job layout");

#define DITK_REQUIRE(cond, ...)        \
  do {                                 \
    if (!(cond)) {                     \
      ditk_set_error(__VA_ARGS__);     \
      return 1;                        \
    }                                  \
  } while (0)

// ---------------------------------------------------------------------------
// bf16 <-> fp32 (device)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;

// fp32 -> bf16, round to nearest even (gfx950 v_cvt_pk_bf16_f32)
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// round an fp32 value to the nearest bf16 and return it as fp32
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  bf16x2_t v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// unpack 8 bf16 held in a 16-byte vector
__device__ __forceinline__ void unpack8(const u32x4_t v, float* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(v[i] << 16);
    out[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ u32x4_t pack8(const float* in) {
  u32x4_t v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_bf2(in[2 * i], in[2 * i + 1]);
  return v;
}

// ---------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------
template <int WIDTH>
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int WIDTH>
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// segment of token t in cu[0..nseg] (cu[0] = 0, nondecreasing); tokens at or
// beyond cu[nseg] map to nseg - 1.
__device__ __forceinline__ int find_segment(const int32_t* __restrict__ cu, int nseg, int t) {
  int lo = 0, hi = nseg - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__device__ __forceinline__ float gelu_tanh_f(float x) {
  // 0.5 x (1 + tanh(u)) == x / (1 + exp(-2u)),  u = sqrt(2/pi) (x + 0.044715 x^3);
  // exp(-2u) = 2^(x (C0 + C1 x^2)) with C0 = -2 sqrt(2/pi) / ln 2, C1 = 0.044715 C0.
  // v_exp_f32 and v_rcp_f32 (1 ulp each) are far below the bf16 output rounding;
  // for x -> -inf the power overflows to inf and the result is -0.
  const float C0 = -2.3022082f, C1 = -0.10294324f;
  const float e = __builtin_amdgcn_exp2f(x * fmaf(x * x, C1, C0));
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float silu_f(float x) {
  // x / (1 + e^-x), e^-x = 2^(-x / ln 2)
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950f));
}
