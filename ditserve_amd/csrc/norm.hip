// Row-normalisation kernels: fused AdaLN (LayerNorm/RMSNorm + per-segment
// shift/scale modulation), the modulation table add, and the fused
// QK-RMSNorm + 3D RoPE kernel.
//
// All three are HBM-bound: one wave64 owns one token row, keeps the row in
// registers (8 bf16 per 16-byte load per lane), reduces with wave shuffles and
// writes the row once.  Per-token results depend only on the row and its
// segment's modulation, so packed and per-request runs agree bitwise.
#include "ditk_common.h"

namespace {

constexpr int kRowsPerBlock = 4;  // 4 waves, one row each
constexpr int kMaxChunks = 12;    // 16-byte chunks per lane -> D <= 64*8*12 = 6144

// ---------------------------------------------------------------------------
// AdaLN:  y = norm(x) [* w + b] [* (1 + scale[seg]) + shift[seg]]
//   norm = LayerNorm (kind 0) or RMSNorm (kind 1), eps inside the rsqrt.
// ---------------------------------------------------------------------------
// AFF: an unmodulated row with affine weight and/or bias, whose vectors are
// then loaded before the reductions like the modulation (a variant of its own,
// so that the modulated kernels keep their register allocation).
template <int KIND, int NC, bool AFF = false>
__device__ __forceinline__ void adaln_row(
    const bf16_t* __restrict__ x, int64_t ldx, bf16_t* __restrict__ y, int64_t ldy, int row, int D,
    const int32_t* __restrict__ cu, int nseg, const float* __restrict__ shift,
    const float* __restrict__ scale, int64_t mod_stride, const float* __restrict__ w,
    const float* __restrict__ b, float eps) {
  const int lane = threadIdx.x & 63;
  const int nchunk = D >> 3;
  const bf16_t* xr = x + (int64_t)row * ldx;
  // Every load of the row is issued before the reductions: the row itself
  // (NC 16-byte chunks per lane, kept packed), then its segment's scale and
  // shift or, unmodulated, the affine weight and bias (L2-resident), so the
  // latencies overlap.
  u32x4_t raw[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = i * 64 + lane;
    raw[i] = c < nchunk ? *reinterpret_cast<const u32x4_t*>(xr + c * 8) : u32x4_t{0, 0, 0, 0};
  }
  f32x4_t sc4[NC][2], sh4[NC][2];
  const bool mod = !AFF && shift != nullptr;
  // AFF rows hold the affine vectors in the modulation's registers: sc4 = w, sh4 = b
  constexpr bool aff_pre = AFF;
  if (aff_pre) {
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = min(i * 64 + lane, nchunk - 1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        sc4[i][h] = w != nullptr ? *reinterpret_cast<const f32x4_t*>(w + c * 8 + 4 * h) : f32x4_t{1.f, 1.f, 1.f, 1.f};
        sh4[i][h] = b != nullptr ? *reinterpret_cast<const f32x4_t*>(b + c * 8 + 4 * h) : f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
    }
  }
  if (mod) {
    const int seg = find_segment(cu, nseg, row);
    const float* sh = shift + (int64_t)seg * mod_stride;
    const float* sc = scale + (int64_t)seg * mod_stride;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = min(i * 64 + lane, nchunk - 1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        sc4[i][h] = *reinterpret_cast<const f32x4_t*>(sc + c * 8 + 4 * h);
        sh4[i][h] = *reinterpret_cast<const f32x4_t*>(sh + c * 8 + 4 * h);
      }
    }
  }
  float mean = 0.f;
  if (KIND == 0) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      float v[8];
      unpack8(raw[i], v);
#pragma unroll
      for (int j = 0; j < 8; ++j) s += v[j];
    }
    mean = wave_sum<64>(s) / (float)D;
  }
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    if (i * 64 + lane < nchunk) {
      float v[8];
      unpack8(raw[i], v);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float d = v[j] - mean;
        q = fmaf(d, d, q);
      }
    }
  }
  const float rstd = rsqrtf(wave_sum<64>(q) / (float)D + eps);
  bf16_t* yr = y + (int64_t)row * ldy;
  // affine vectors (not on the modulated path) are read as two 16-byte loads per chunk
  auto load8 = [](const float* p, float* out) {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(p);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(p + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      out[j] = a[j];
      out[j + 4] = b[j];
    }
  };
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = i * 64 + lane;
    if (c < nchunk) {
      float o[8], t[8];
      unpack8(raw[i], o);
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = (o[j] - mean) * rstd;
      if (aff_pre) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (w != nullptr) {
            o[j] *= sc4[i][0][j];
            o[j + 4] *= sc4[i][1][j];
          }
          if (b != nullptr) {
            o[j] += sh4[i][0][j];
            o[j + 4] += sh4[i][1][j];
          }
        }
      } else if (w != nullptr) {
        load8(w + c * 8, t);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] *= t[j];
      }
      if (!aff_pre && b != nullptr) {
        load8(b + c * 8, t);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] += t[j];
      }
      if (mod) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          o[j] = o[j] * (1.0f + sc4[i][0][j]) + sh4[i][0][j];
          o[j + 4] = o[j + 4] * (1.0f + sc4[i][1][j]) + sh4[i][1][j];
        }
      }
      *reinterpret_cast<u32x4_t*>(yr + c * 8) = pack8(o);
    }
  }
}

template <int KIND, int NC, bool AFF>
__global__ __launch_bounds__(256) void adaln_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, bf16_t* __restrict__ y, int64_t ldy, int T, int D,
    const int32_t* __restrict__ cu, int nseg, const float* __restrict__ shift,
    const float* __restrict__ scale, int64_t mod_stride, const float* __restrict__ w,
    const float* __restrict__ b, float eps) {
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= T) return;
  adaln_row<KIND, NC, AFF>(x, ldx, y, ldy, row, D, cu, nseg, shift, scale, mod_stride, w, b, eps);
}

// Several AdaLN jobs of one norm kind and chunk count in one launch: job j owns
// workgroups [block0[j], block0[j + 1]), four rows each, and runs adaln_row on
// its own tensors, so each row is computed exactly as a single-job launch would.
constexpr int kMaxJobs = 4;
struct AdalnJob {
  const bf16_t* x;
  int64_t ldx;
  bf16_t* y;
  int64_t ldy;
  const int32_t* cu;
  const float* shift;
  const float* scale;
  int64_t mod_stride;
  const float* w;
  const float* b;
  int T, D, nseg;
  float eps;
};
struct AdalnJobs {
  AdalnJob job[kMaxJobs];
  int block0[kMaxJobs + 1];
  int njobs;
};

template <int KIND, int NC, bool AFF>
__global__ __launch_bounds__(256) void adaln_multi_kernel(AdalnJobs jobs) {
  int j = 0;
  while (j + 1 < jobs.njobs && (int)blockIdx.x >= jobs.block0[j + 1]) ++j;
  const AdalnJob& a = jobs.job[j];
  const int row = ((int)blockIdx.x - jobs.block0[j]) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= a.T) return;
  adaln_row<KIND, NC, AFF>(a.x, a.ldx, a.y, a.ldy, row, a.D, a.cu, a.nseg, a.shift, a.scale, a.mod_stride, a.w, a.b,
                      a.eps);
}

// mod[s, j, d] = table[j, d] + proj[s, j, d]   (fp32; k rows of D per segment)
__global__ void modulation_kernel(const float* __restrict__ table, const float* __restrict__ proj,
                                  float* __restrict__ mod, int nseg, int kd) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t n = (int64_t)nseg * kd;
  if (i < n) mod[i] = table[i % kd] + proj[i];
}

// ---------------------------------------------------------------------------
// QK RMSNorm (+ 3D RoPE), in place.
//   group == D : RMSNorm across all heads (Wan "rms_norm_across_heads")
//   group == head_dim : per-head RMSNorm (SD3.5 "rms_norm")
// RoPE (optional): pair p of each head rotates by the angle of the token's
// position on the axis that owns p: p < t_pairs -> frame, p < t_pairs+h_pairs
// -> row, else column.  Angles come from cos/sin tables [max_pos][head_dim/2]
// built in float64 and rounded to fp32 on the host.
// Work item: one wave per token, normalising its q row and its k row, so the
// segment search, the position arithmetic and the rotation's table loads are
// shared by both.  Every address computation stays in registers (positions are
// selected by value), so the kernel uses no scratch or LDS.
// ---------------------------------------------------------------------------
template <int NC>
__device__ __forceinline__ void load_w(const float* __restrict__ w, int nchunk, int lane, f32x4_t (&w4)[NC][2]) {
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = min(i * 64 + lane, nchunk - 1);
    w4[i][0] = *reinterpret_cast<const f32x4_t*>(w + c * 8);
    w4[i][1] = *reinterpret_cast<const f32x4_t*>(w + c * 8 + 4);
  }
}

// reciprocal RMS of each chunk's group (one value per chunk; equal across a
// wave when the group is the whole row)
template <int GROUP_LANES, int NC>
__device__ __forceinline__ void group_rstd(const u32x4_t (&raw)[NC], int D, int head_dim, float eps,
                                           float (&rs)[NC]) {
  float ss[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    float v[8];
    unpack8(raw[i], v);
    ss[i] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss[i] = fmaf(v[j], v[j], ss[i]);
  }
  if (GROUP_LANES == 64) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) t += ss[i];
    const float r = rsqrtf(wave_sum<64>(t) / (float)D + eps);
#pragma unroll
    for (int i = 0; i < NC; ++i) rs[i] = r;
  } else {
    // a head spans GROUP_LANES consecutive lanes of one chunk row
#pragma unroll
    for (int i = 0; i < NC; ++i) rs[i] = rsqrtf(wave_sum<GROUP_LANES>(ss[i]) / (float)head_dim + eps);
  }
}

template <int NC>
__device__ __forceinline__ void norm_rotate_store(bf16_t* __restrict__ xr, const u32x4_t (&raw)[NC],
                                                  const float (&rs)[NC], const f32x4_t (&w4)[NC][2],
                                                  bool rope, const float (&rc)[4], const float (&rsn)[4],
                                                  int nchunk, int lane) {
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = i * 64 + lane;
    if (c < nchunk) {
      float o[8];
      unpack8(raw[i], o);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        o[j] = o[j] * rs[i] * w4[i][0][j];
        o[j + 4] = o[j + 4] * rs[i] * w4[i][1][j];
      }
      if (rope) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x1 = o[2 * j], x2 = o[2 * j + 1];
          o[2 * j] = x1 * rc[j] - x2 * rsn[j];
          o[2 * j + 1] = x1 * rsn[j] + x2 * rc[j];
        }
      }
      *reinterpret_cast<u32x4_t*>(xr + c * 8) = pack8(o);
    }
  }
}

template <int GROUP_LANES, int NC>
__device__ __forceinline__ void qk_norm_row(
    const bf16_t* q, int64_t ldq, const bf16_t* k, int64_t ldk, bf16_t* qo, int64_t ldqo, bf16_t* ko,
    int64_t ldko, int row, int D,
    int head_dim, const float* __restrict__ wq, const float* __restrict__ wk, float eps,
    const float* __restrict__ rcos, const float* __restrict__ rsin, int max_pos,
    const int32_t* __restrict__ cu, const int32_t* __restrict__ grids, int nseg, int t_pairs,
    int h_pairs) {
  // Norm weights are L2-resident; up to 4 chunks per lane they are loaded with
  // the rows (before the reductions), above that after them to bound registers.
  constexpr bool kEarlyW = NC <= 4;
  const int lane = threadIdx.x & 63;
  // q/k may be the outputs themselves (in place): a lane reads its row chunks
  // before it writes them, and no other lane touches them
  const bf16_t* qr = q + (int64_t)row * ldq;
  const bf16_t* kr = k + (int64_t)row * ldk;
  const int nchunk = D >> 3;
  u32x4_t rawq[NC], rawk[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = i * 64 + lane;
    rawq[i] = c < nchunk ? *reinterpret_cast<const u32x4_t*>(qr + c * 8) : u32x4_t{0, 0, 0, 0};
    rawk[i] = c < nchunk ? *reinterpret_cast<const u32x4_t*>(kr + c * 8) : u32x4_t{0, 0, 0, 0};
  }
  f32x4_t wq4[NC][2], wk4[NC][2];
  if (kEarlyW) {
    load_w<NC>(wq, nchunk, lane, wq4);
    load_w<NC>(wk, nchunk, lane, wk4);
  }
  // RoPE: chunk c holds pairs p0..p0+3 of its head, p0 = 4 * (c % (head_dim/8));
  // with 64 lanes per chunk row that is the same quad for every chunk of a lane,
  // so each lane loads its rotation once, for q and k together.  The quad's
  // pairs belong to at most two axes: table entries of the axis of the first
  // pair and of the last pair.
  const bool rope = rcos != nullptr;
  const int p0 = (lane % (head_dim >> 3)) * 4;
  float rc[4] = {1.f, 1.f, 1.f, 1.f}, rsn[4] = {0.f, 0.f, 0.f, 0.f};
  if (rope) {
    const int half = head_dim >> 1;
    const int seg = find_segment(cu, nseg, row);
    const int s = row - cu[seg];
    const int gh = grids[seg * 3 + 1], gw = grids[seg * 3 + 2];
    const int pf = min(s / (gh * gw), max_pos - 1);
    const int ph = min((s / gw) % gh, max_pos - 1);
    const int pw = min(s % gw, max_pos - 1);
    const int th = t_pairs + h_pairs;
    const int pa = p0 < t_pairs ? pf : (p0 < th ? ph : pw);
    const int pb = p0 + 3 < t_pairs ? pf : (p0 + 3 < th ? ph : pw);
    const f32x4_t ca = *reinterpret_cast<const f32x4_t*>(rcos + pa * half + p0);
    const f32x4_t sa = *reinterpret_cast<const f32x4_t*>(rsin + pa * half + p0);
    const f32x4_t cb = *reinterpret_cast<const f32x4_t*>(rcos + pb * half + p0);
    const f32x4_t sb = *reinterpret_cast<const f32x4_t*>(rsin + pb * half + p0);
    const bool a_t = p0 < t_pairs, a_h = p0 < th;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool first = ((p0 + j < t_pairs) == a_t) && ((p0 + j < th) == a_h);
      rc[j] = first ? ca[j] : cb[j];
      rsn[j] = first ? sa[j] : sb[j];
    }
  }
  float rsq[NC], rsk[NC];
  group_rstd<GROUP_LANES, NC>(rawq, D, head_dim, eps, rsq);
  group_rstd<GROUP_LANES, NC>(rawk, D, head_dim, eps, rsk);
  if (!kEarlyW) {
    load_w<NC>(wq, nchunk, lane, wq4);
    load_w<NC>(wk, nchunk, lane, wk4);
  }
  norm_rotate_store<NC>(qo + (int64_t)row * ldqo, rawq, rsq, wq4, rope, rc, rsn, nchunk, lane);
  norm_rotate_store<NC>(ko + (int64_t)row * ldko, rawk, rsk, wk4, rope, rc, rsn, nchunk, lane);
}

template <int GROUP_LANES, int NC>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const bf16_t* q, int64_t ldq, const bf16_t* k, int64_t ldk, bf16_t* qo, int64_t ldqo, bf16_t* ko,
    int64_t ldko, int T, int D,
    int head_dim, const float* __restrict__ wq, const float* __restrict__ wk, float eps,
    const float* __restrict__ rcos, const float* __restrict__ rsin, int max_pos,
    const int32_t* __restrict__ cu, const int32_t* __restrict__ grids, int nseg, int t_pairs,
    int h_pairs) {
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= T) return;
  qk_norm_row<GROUP_LANES, NC>(q, ldq, k, ldk, qo, ldqo, ko, ldko, row, D, head_dim, wq, wk, eps, rcos, rsin,
                               max_pos, cu, grids, nseg, t_pairs, h_pairs);
}

// Several RoPE-free QK-norm jobs of one group width and chunk count in one
// launch (SD3.5's image and text per-head norms): job j owns workgroups
// [block0[j], block0[j + 1]) and runs qk_norm_row on its own tensors.
struct QkNormJobs {
  ditk_qk_norm_job job[kMaxJobs];
  int block0[kMaxJobs + 1];
  int njobs;
};

template <int GROUP_LANES, int NC>
__global__ __launch_bounds__(256) void qk_norm_multi_kernel(QkNormJobs jobs) {
  int j = 0;
  while (j + 1 < jobs.njobs && (int)blockIdx.x >= jobs.block0[j + 1]) ++j;
  const ditk_qk_norm_job& a = jobs.job[j];
  const int row = ((int)blockIdx.x - jobs.block0[j]) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= a.T) return;
  qk_norm_row<GROUP_LANES, NC>((const bf16_t*)a.q, a.ldq, (const bf16_t*)a.k, a.ldk, (bf16_t*)a.q_out, a.ldqo,
                               (bf16_t*)a.k_out, a.ldko, row, a.D, a.head_dim, a.wq, a.wk, a.eps, nullptr, nullptr,
                               0, nullptr, nullptr, 0, 0, 0);
}

}  // namespace

namespace {
int adaln_check(const void* x, int64_t ldx, void* y, int64_t ldy, int T, int D, const int32_t* cu_seqlens, int nseg,
                const float* shift, const float* scale, int64_t mod_stride, const float* weight, const float* bias,
                int norm_kind) {
  DITK_REQUIRE(T == 0 || (x != nullptr && y != nullptr), "ditk_adaln: null tensor");
  DITK_REQUIRE(T >= 0 && D > 0 && D % 8 == 0 && D <= 64 * 8 * kMaxChunks,
               "ditk_adaln: D=%d must be a positive multiple of 8 and <= %d", D, 64 * 8 * kMaxChunks);
  DITK_REQUIRE(ldx % 8 == 0 && ldy % 8 == 0 && ldx >= D && ldy >= D,
               "ditk_adaln: leading dims must be multiples of 8 and >= D");
  DITK_REQUIRE((shift == nullptr) == (scale == nullptr), "ditk_adaln: shift and scale go together");
  DITK_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0, "ditk_adaln: x and y must be 16-byte aligned");
  DITK_REQUIRE(((uintptr_t)shift % 16) == 0 && ((uintptr_t)scale % 16) == 0 && mod_stride % 4 == 0 &&
               ((uintptr_t)weight % 16) == 0 && ((uintptr_t)bias % 16) == 0,
               "ditk_adaln: modulation / affine vectors must be 16-byte aligned");
  DITK_REQUIRE(shift == nullptr || (cu_seqlens != nullptr && nseg > 0),
               "ditk_adaln: modulation needs cu_seqlens");
  DITK_REQUIRE(norm_kind == 0 || norm_kind == 1, "ditk_adaln: norm_kind must be 0 (LN) or 1 (RMS)");
  return 0;
}
}  // namespace

DITK_EXPORT int ditk_adaln(const void* x, int64_t ldx, void* y, int64_t ldy, int T, int D,
                           const int32_t* cu_seqlens, int nseg, const float* shift,
                           const float* scale, int64_t mod_stride, const float* weight,
                           const float* bias, float eps, int norm_kind, hipStream_t stream) {
  const int rc = adaln_check(x, ldx, y, ldy, T, D, cu_seqlens, nseg, shift, scale, mod_stride, weight, bias,
                             norm_kind);
  if (rc) return rc;
  if (T == 0) return 0;
  dim3 grid((T + kRowsPerBlock - 1) / kRowsPerBlock);
  const int nc = (D / 8 + 63) / 64;
  const bool aff = shift == nullptr && (weight != nullptr || bias != nullptr);
#define DITK_ADALN(K, NCV)                                                                                     \
  (aff ? adaln_kernel<K, NCV, true> : adaln_kernel<K, NCV, false>)<<<grid, 256, 0, stream>>>(                  \
      (const bf16_t*)x, ldx, (bf16_t*)y, ldy, T, D, cu_seqlens, nseg, shift, scale, mod_stride, weight, bias, eps)
#define DITK_ADALN_NC(K)              \
  switch (nc) {                       \
    case 1: DITK_ADALN(K, 1); break;  \
    case 2: DITK_ADALN(K, 2); break;  \
    case 3: DITK_ADALN(K, 3); break;  \
    case 4: DITK_ADALN(K, 4); break;  \
    case 5: DITK_ADALN(K, 5); break;  \
    case 6: DITK_ADALN(K, 6); break;  \
    case 7: DITK_ADALN(K, 7); break;  \
    case 8: DITK_ADALN(K, 8); break;   \
    case 9:                         \
    case 10: DITK_ADALN(K, 10); break; \
    default: DITK_ADALN(K, 12); break; \
  }
  if (norm_kind == 0) {
    DITK_ADALN_NC(0)
  } else {
    DITK_ADALN_NC(1)
  }
#undef DITK_ADALN_NC
#undef DITK_ADALN
  return ditk_check_launch("ditk_adaln");
}

DITK_EXPORT int ditk_adaln_multi(const ditk_adaln_job* jobs, int njobs, hipStream_t stream) {
  DITK_REQUIRE(jobs != nullptr && njobs >= 1 && njobs <= kMaxJobs, "ditk_adaln_multi: 1 to %d jobs", kMaxJobs);
  AdalnJobs a = {};
  a.njobs = njobs;
  int nc = 0, kind = 0;
  bool aff = true;  // every job unmodulated with affine vectors
  int64_t blocks = 0;
  for (int j = 0; j < njobs; ++j) {
    const ditk_adaln_job& p = jobs[j];
    aff = aff && p.shift == nullptr && (p.weight != nullptr || p.bias != nullptr);
    const int rc = adaln_check(p.x, p.ldx, p.y, p.ldy, p.T, p.D, p.cu_seqlens, p.nseg, p.shift, p.scale,
                               p.mod_stride, p.weight, p.bias, p.norm_kind);
    if (rc) return rc;
    const int ncj = (p.D / 8 + 63) / 64;
    DITK_REQUIRE(j == 0 || (ncj == nc && p.norm_kind == kind),
                 "ditk_adaln_multi: jobs must share the norm kind and ceil(D / 512)");
    nc = ncj;
    kind = p.norm_kind;
    a.job[j] = AdalnJob{(const bf16_t*)p.x, p.ldx, (bf16_t*)p.y, p.ldy, p.cu_seqlens, p.shift, p.scale,
                        p.mod_stride, p.weight, p.bias, p.T, p.D, p.nseg, p.eps};
    a.block0[j] = (int)blocks;
    blocks += (p.T + kRowsPerBlock - 1) / kRowsPerBlock;
  }
  DITK_REQUIRE(blocks < (1ll << 31), "ditk_adaln_multi: too many rows");
  a.block0[njobs] = (int)blocks;
  if (blocks == 0) return 0;
  const dim3 grid((unsigned)blocks);
#define DITK_ADALN_M(K, NCV) \
  (aff ? adaln_multi_kernel<K, NCV, true> : adaln_multi_kernel<K, NCV, false>)<<<grid, 256, 0, stream>>>(a)
#define DITK_ADALN_M_NC(K)              \
  switch (nc) {                         \
    case 1: DITK_ADALN_M(K, 1); break;  \
    case 2: DITK_ADALN_M(K, 2); break;  \
    case 3: DITK_ADALN_M(K, 3); break;  \
    case 4: DITK_ADALN_M(K, 4); break;  \
    case 5: DITK_ADALN_M(K, 5); break;  \
    case 6: DITK_ADALN_M(K, 6); break;  \
    case 7: DITK_ADALN_M(K, 7); break;  \
    case 8: DITK_ADALN_M(K, 8); break;   \
    case 9:                         \
    case 10: DITK_ADALN_M(K, 10); break; \
    default: DITK_ADALN_M(K, 12); break; \
  }
  if (kind == 0) {
    DITK_ADALN_M_NC(0)
  } else {
    DITK_ADALN_M_NC(1)
  }
#undef DITK_ADALN_M_NC
#undef DITK_ADALN_M
  return ditk_check_launch("ditk_adaln_multi");
}

DITK_EXPORT int ditk_modulation(const float* table, const float* proj, float* mod, int nseg, int kd,
                                hipStream_t stream) {
  DITK_REQUIRE(table && proj && mod && nseg > 0 && kd > 0, "ditk_modulation: bad arguments");
  int64_t n = (int64_t)nseg * kd;
  modulation_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(table, proj, mod, nseg, kd);
  return ditk_check_launch("ditk_modulation");
}

namespace {
int qk_norm_check(const void* q, int64_t ldq, const void* k, int64_t ldk, void* qo, int64_t ldqo, void* ko,
                  int64_t ldko, int T, int D, int head_dim, const float* wq, const float* wk, const float* rope_cos,
                  const float* rope_sin, int max_pos, const int32_t* cu_seqlens, const int32_t* grids, int nseg,
                  int t_pairs, int h_pairs) {
  DITK_REQUIRE(T >= 0, "ditk_qk_norm_rope: bad T");
  // the row tensors may be NULL when there are no rows
  DITK_REQUIRE((T == 0 || (q && k && qo && ko)) && wq && wk, "ditk_qk_norm_rope: null tensor");
  DITK_REQUIRE(D > 0 && D % 8 == 0 && D <= 64 * 8 * kMaxChunks, "ditk_qk_norm_rope: bad D=%d", D);
  DITK_REQUIRE(head_dim == 64 || head_dim == 128, "ditk_qk_norm_rope: head_dim must be 64 or 128");
  DITK_REQUIRE(D % head_dim == 0, "ditk_qk_norm_rope: D %% head_dim != 0");
  DITK_REQUIRE(ldq % 8 == 0 && ldk % 8 == 0 && ldqo % 8 == 0 && ldko % 8 == 0,
               "ditk_qk_norm_rope: leading dims must be multiples of 8");
  DITK_REQUIRE(((uintptr_t)qo % 16) == 0 && ((uintptr_t)ko % 16) == 0, "ditk_qk_norm_rope: outputs must be 16-byte aligned");
  DITK_REQUIRE(((uintptr_t)q % 16) == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)wq % 16) == 0 &&
               ((uintptr_t)wk % 16) == 0, "ditk_qk_norm_rope: tensors must be 16-byte aligned");
  DITK_REQUIRE(rope_cos == nullptr || (rope_sin && cu_seqlens && grids && nseg > 0 && max_pos > 0),
               "ditk_qk_norm_rope: RoPE needs tables, cu_seqlens and grids");
  DITK_REQUIRE(rope_cos == nullptr || (t_pairs >= 0 && h_pairs >= 0 && t_pairs + h_pairs <= head_dim / 2),
               "ditk_qk_norm_rope: bad axis split");
  DITK_REQUIRE(rope_cos == nullptr || h_pairs == 0 || h_pairs >= 4,
               "ditk_qk_norm_rope: the middle axis must own 0 or >= 4 pairs");
  DITK_REQUIRE(rope_cos == nullptr || (((uintptr_t)rope_cos % 16) == 0 && ((uintptr_t)rope_sin % 16) == 0),
               "ditk_qk_norm_rope: RoPE tables must be 16-byte aligned");
  return 0;
}

int qk_norm_rope_launch(const void* q, int64_t ldq, const void* k, int64_t ldk, void* qo, int64_t ldqo, void* ko,
                        int64_t ldko, int T, int D, int head_dim, const float* wq, const float* wk, float eps,
                        int per_head, const float* rope_cos, const float* rope_sin, int max_pos,
                        const int32_t* cu_seqlens, const int32_t* grids, int nseg, int t_pairs, int h_pairs,
                        hipStream_t stream) {
  const int rc = qk_norm_check(q, ldq, k, ldk, qo, ldqo, ko, ldko, T, D, head_dim, wq, wk, rope_cos, rope_sin,
                               max_pos, cu_seqlens, grids, nseg, t_pairs, h_pairs);
  if (rc) return rc;
  if (T == 0) return 0;
  dim3 grid((T + kRowsPerBlock - 1) / kRowsPerBlock);
  const int nc = (D / 8 + 63) / 64;
#define DITK_QKN(G, NCV)                                                                                  \
  qk_norm_rope_kernel<G, NCV><<<grid, 256, 0, stream>>>((const bf16_t*)q, ldq, (const bf16_t*)k, ldk,    \
                                                        (bf16_t*)qo, ldqo, (bf16_t*)ko, ldko, T, D, head_dim, \
                                                        wq, wk, eps, rope_cos, rope_sin, max_pos,         \
                                                        cu_seqlens, grids, nseg, t_pairs, h_pairs)
#define DITK_QKN_NC(G)              \
  switch (nc) {                     \
    case 1: DITK_QKN(G, 1); break;  \
    case 2: DITK_QKN(G, 2); break;  \
    case 3: DITK_QKN(G, 3); break;  \
    case 4: DITK_QKN(G, 4); break;  \
    case 5: DITK_QKN(G, 5); break;  \
    case 6: DITK_QKN(G, 6); break;  \
    case 7: DITK_QKN(G, 7); break;  \
    case 8: DITK_QKN(G, 8); break;   \
    case 9:                         \
    case 10: DITK_QKN(G, 10); break; \
    default: DITK_QKN(G, 12); break; \
  }
  if (!per_head) {
    DITK_QKN_NC(64)
  } else if (head_dim == 128) {
    DITK_QKN_NC(16)
  } else {
    DITK_QKN_NC(8)
  }
#undef DITK_QKN_NC
#undef DITK_QKN
  return ditk_check_launch("ditk_qk_norm_rope");
}
}  // namespace

DITK_EXPORT int ditk_qk_norm_multi(const ditk_qk_norm_job* jobs, int njobs, hipStream_t stream) {
  DITK_REQUIRE(jobs != nullptr && njobs >= 1 && njobs <= kMaxJobs, "ditk_qk_norm_multi: 1 to %d jobs", kMaxJobs);
  QkNormJobs a = {};
  a.njobs = njobs;
  int nc = 0, group = 0;
  int64_t blocks = 0;
  for (int j = 0; j < njobs; ++j) {
    const ditk_qk_norm_job& p = jobs[j];
    const int rc = qk_norm_check(p.q, p.ldq, p.k, p.ldk, p.q_out, p.ldqo, p.k_out, p.ldko, p.T, p.D, p.head_dim, p.wq,
                                 p.wk, nullptr, nullptr, 0, nullptr, nullptr, 0, 0, 0);
    if (rc) return rc;
    const int ncj = (p.D / 8 + 63) / 64;
    const int gj = !p.per_head ? 64 : (p.head_dim == 128 ? 16 : 8);
    DITK_REQUIRE(j == 0 || (ncj == nc && gj == group),
                 "ditk_qk_norm_multi: jobs must share ceil(D / 512) and the norm grouping (per head and head_dim)");
    nc = ncj;
    group = gj;
    a.job[j] = p;
    a.block0[j] = (int)blocks;
    blocks += (p.T + kRowsPerBlock - 1) / kRowsPerBlock;
  }
  DITK_REQUIRE(blocks < (1ll << 31), "ditk_qk_norm_multi: too many rows");
  a.block0[njobs] = (int)blocks;
  if (blocks == 0) return 0;
  const dim3 grid((unsigned)blocks);
#define DITK_QKM(G, NCV) qk_norm_multi_kernel<G, NCV><<<grid, 256, 0, stream>>>(a)
#define DITK_QKM_NC(G)              \
  switch (nc) {                     \
    case 1: DITK_QKM(G, 1); break;  \
    case 2: DITK_QKM(G, 2); break;  \
    case 3: DITK_QKM(G, 3); break;  \
    case 4: DITK_QKM(G, 4); break;  \
    case 5: DITK_QKM(G, 5); break;  \
    case 6: DITK_QKM(G, 6); break;  \
    case 7: DITK_QKM(G, 7); break;  \
    case 8: DITK_QKM(G, 8); break;   \
    case 9:                         \
    case 10: DITK_QKM(G, 10); break; \
    default: DITK_QKM(G, 12); break; \
  }
  if (group == 64) {
    DITK_QKM_NC(64)
  } else if (group == 16) {
    DITK_QKM_NC(16)
  } else {
    DITK_QKM_NC(8)
  }
#undef DITK_QKM_NC
#undef DITK_QKM
  return ditk_check_launch("ditk_qk_norm_multi");
}

DITK_EXPORT int ditk_qk_norm_rope(void* q, int64_t ldq, void* k, int64_t ldk, int T, int D,
                                  int head_dim, const float* wq, const float* wk, float eps,
                                  int per_head, const float* rope_cos, const float* rope_sin,
                                  int max_pos, const int32_t* cu_seqlens, const int32_t* grids,
                                  int nseg, int t_pairs, int h_pairs, hipStream_t stream) {
  return qk_norm_rope_launch(q, ldq, k, ldk, q, ldq, k, ldk, T, D, head_dim, wq, wk, eps, per_head, rope_cos,
                             rope_sin, max_pos, cu_seqlens, grids, nseg, t_pairs, h_pairs, stream);
}

DITK_EXPORT int ditk_qk_norm_rope_out(const void* q, int64_t ldq, const void* k, int64_t ldk, void* q_out,
                                      int64_t ldqo, void* k_out, int64_t ldko, int T, int D, int head_dim,
                                      const float* wq, const float* wk, float eps, int per_head,
                                      const float* rope_cos, const float* rope_sin, int max_pos,
                                      const int32_t* cu_seqlens, const int32_t* grids, int nseg, int t_pairs,
                                      int h_pairs, hipStream_t stream) {
  return qk_norm_rope_launch(q, ldq, k, ldk, q_out, ldqo, k_out, ldko, T, D, head_dim, wq, wk, eps, per_head,
                             rope_cos, rope_sin, max_pos, cu_seqlens, grids, nseg, t_pairs, h_pairs, stream);
}
