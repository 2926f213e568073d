// Bandwidth-bound glue of the packet prelude / epilogue and of SD3.5 joint
// attention: patchify, unpatchify, sinusoidal timestep embedding, CFG combine,
// joint-sequence gather / scatter.  Each is a plain coalesced elementwise pass.
#include <math.h>

#include "ditk_common.h"

namespace {

// latent [C, F, H, W] (bf16) -> patches [S, C*pt*ph*pw] (bf16), token order
// f-major, then h, then w; patch vector order (c, i, j, l) as a Conv3d weight.
__global__ void patchify_kernel(const bf16_t* __restrict__ lat, bf16_t* __restrict__ out, int C, int F,
                                int H, int W, int pt, int ph, int pw) {
  const int Fp = F / pt, Hp = H / ph, Wp = W / pw;
  const int P = C * pt * ph * pw;
  const int64_t n = (int64_t)Fp * Hp * Wp * P;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
       idx += (int64_t)gridDim.x * blockDim.x) {
    int64_t s = idx / P;
    int p = (int)(idx % P);
    int c = p / (pt * ph * pw), r = p % (pt * ph * pw);
    int i = r / (ph * pw), j = (r / pw) % ph, l = r % pw;
    int f = (int)(s / ((int64_t)Hp * Wp)), hh = (int)((s / Wp) % Hp), ww = (int)(s % Wp);
    out[idx] = lat[(((int64_t)c * F + f * pt + i) * H + hh * ph + j) * W + ww * pw + l];
  }
}

// x [S, pt*ph*pw*C] (bf16, feature order (i, j, l, c)) -> latent [C, F, H, W] (fp32)
__global__ void unpatchify_kernel(const bf16_t* __restrict__ x, int64_t ldx, float* __restrict__ out,
                                  int C, int Fp, int Hp, int Wp, int pt, int ph, int pw) {
  const int F = Fp * pt, H = Hp * ph, W = Wp * pw;
  const int64_t n = (int64_t)C * F * H * W;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
       idx += (int64_t)gridDim.x * blockDim.x) {
    int w = (int)(idx % W);
    int h = (int)((idx / W) % H);
    int f = (int)((idx / ((int64_t)W * H)) % F);
    int c = (int)(idx / ((int64_t)W * H * F));
    int64_t s = ((int64_t)(f / pt) * Hp + h / ph) * Wp + w / pw;
    int feat = (((f % pt) * ph + h % ph) * pw + w % pw) * C + c;
    out[idx] = bf2f(x[s * ldx + feat]);
  }
}

// emb[n, :] = [cos(t_n * f_k), sin(t_n * f_k)],  f_k = exp(-ln(max_period) * k / half)
// (flip_sin_to_cos ordering, frequency shift 0), bf16 out.
__global__ void timestep_embed_kernel(const float* __restrict__ t, bf16_t* __restrict__ out, int N, int dim,
                                      float log_max_period) {
  const int half = dim / 2;
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)N * dim) return;
  int n = (int)(idx / dim), k = (int)(idx % dim);
  int kk = k % half;
  float freq = expf(-log_max_period * (float)kk / (float)half);
  float a = t[n] * freq;
  out[idx] = f2bf(k < half ? cosf(a) : sinf(a));
}

// out = u + g * (c - u)
__global__ void cfg_combine_kernel(const float* __restrict__ cond, const float* __restrict__ uncond,
                                   float* __restrict__ out, int64_t n, float g) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = uncond[i] + g * (cond[i] - uncond[i]);
}

// Fused CFG combine + solver step over one request's latent (fp32), with the
// step's scalar coefficients computed on the host:
//   v  = uncond ? u + g (c - u) : c          CFG combine
//   m  = x - sigma v                          data (x0) prediction of a flow model
//   xc = ax x + a0 xl + a1 mp + a2 mp2 + a3 m corrected sample at sigma
//   xn = b0 xc + b1 m + b2 mp + bv v          predicted sample at the next sigma
// xl / mp / mp2 (last sample, previous two data predictions) are read only when
// their coefficients are non-zero, so they may be null otherwise.  xn may alias x,
// xc may alias xl and m may alias mp2: each element is read before it is written.
struct SolverCoef {
  float g, sigma, ax, a0, a1, a2, a3, b0, b1, b2, bv;
  int use_uncond, use_xl, use_mp, use_mp2;
};

__global__ void solver_step_kernel(const float* x, const float* __restrict__ c,
                                   const float* __restrict__ u, const float* xl, const float* mp,
                                   const float* mp2, float* xn, float* xc_out, float* m_out, int64_t n,
                                   SolverCoef k) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float xi = x[i];
    const float ci = c[i];
    const float v = k.use_uncond ? fmaf(k.g, ci - u[i], u[i]) : ci;
    const float m = fmaf(-k.sigma, v, xi);
    const float xl_i = k.use_xl ? xl[i] : 0.f;
    const float mp_i = k.use_mp ? mp[i] : 0.f;
    const float mp2_i = k.use_mp2 ? mp2[i] : 0.f;
    const float xc = k.ax * xi + k.a0 * xl_i + k.a1 * mp_i + k.a2 * mp2_i + k.a3 * m;
    const float xnext = k.b0 * xc + k.b1 * m + k.b2 * mp_i + k.bv * v;
    if (xc_out) xc_out[i] = xc;
    if (m_out) m_out[i] = m;
    xn[i] = xnext;
  }
}

// joint[cu_joint[m] + r] = img[cu_img[m] + r] for r < n_img(m), then txt rows.
// direction 0: gather (img, txt -> joint); 1: scatter (joint -> img, txt).
__global__ void joint_copy_kernel(bf16_t* __restrict__ img, int64_t ld_img, bf16_t* __restrict__ txt,
                                  int64_t ld_txt, bf16_t* __restrict__ joint, int64_t ld_joint,
                                  const int32_t* __restrict__ cu_img, const int32_t* __restrict__ cu_txt,
                                  int nseg, int total, int width, int direction) {
  const int row = blockIdx.x;
  if (row >= total) return;
  int m = 0;
  {
    int lo = 0, hi = nseg - 1;
    while (lo < hi) {
      int mid = (lo + hi + 1) >> 1;
      if (cu_img[mid] + cu_txt[mid] <= row) lo = mid; else hi = mid - 1;
    }
    m = lo;
  }
  const int r = row - (cu_img[m] + cu_txt[m]);
  const int n_img = cu_img[m + 1] - cu_img[m];
  bf16_t* src = (r < n_img) ? img + (int64_t)(cu_img[m] + r) * ld_img
                            : txt + (int64_t)(cu_txt[m] + r - n_img) * ld_txt;
  bf16_t* j = joint + (int64_t)row * ld_joint;
  for (int c = threadIdx.x; c < width / 8; c += blockDim.x) {
    if (direction == 0)
      reinterpret_cast<u32x4_t*>(j)[c] = reinterpret_cast<const u32x4_t*>(src)[c];
    else
      reinterpret_cast<u32x4_t*>(src)[c] = reinterpret_cast<const u32x4_t*>(j)[c];
  }
}

__global__ void silu_kernel(const bf16_t* __restrict__ x, bf16_t* __restrict__ y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    y[i] = f2bf(silu_f(bf2f(x[i])));
}

inline unsigned grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  return (unsigned)(b > 65536 ? 65536 : (b < 1 ? 1 : b));
}

// A caller's device cu_seqlens table made safe for the segment kernels: out[0] = 0
// and out[i] = max over j <= i of clamp(cu[j], 0, total), so the table is
// nondecreasing inside [0, total] and every row a kernel derives from it exists.
// A valid table (cu[0] = 0, nondecreasing, cu[n-1] = total) comes out unchanged;
// any other sets bit 0 of *status (sticky: this kernel never clears it).  One
// workgroup; chunks of 256 entries, each a block-wide running max on LDS.
__global__ __launch_bounds__(256) void check_cu_kernel(const int32_t* __restrict__ cu, int n, int total,
                                                       int32_t* __restrict__ out, int32_t* __restrict__ status) {
  __shared__ int32_t sm[256];
  const int tid = threadIdx.x;
  int carry = 0, bad = 0;
  for (int base = 0; base < n; base += 256) {
    const int i = base + tid;
    int v = 0;
    if (i < n) {
      const int raw = cu[i];
      const int prev = i > 0 ? cu[i - 1] : 0;
      bad |= (raw < prev) | (raw > total) | (i == 0 && raw != 0) | (i == n - 1 && raw != total);
      v = min(max(raw, 0), total);
    }
    sm[tid] = v;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
      const int x = tid >= off ? sm[tid - off] : 0;
      __syncthreads();
      sm[tid] = max(sm[tid], x);
      __syncthreads();
    }
    if (i < n) out[i] = i == 0 ? 0 : max(sm[tid], carry);
    carry = max(carry, sm[255]);
    __syncthreads();
  }
  if (__syncthreads_or(bad) && tid == 0) atomicOr(status, 1);
}

}  // namespace

DITK_EXPORT int ditk_check_cu_seqlens(const int32_t* cu, int nseg, int total, int32_t* cu_out, int32_t* status,
                                      hipStream_t stream) {
  DITK_REQUIRE(cu && cu_out && status, "ditk_check_cu_seqlens: null pointer");
  DITK_REQUIRE(cu != cu_out, "ditk_check_cu_seqlens: cu_out must not be cu");
  DITK_REQUIRE(nseg > 0 && nseg < (1 << 24) && total >= 0, "ditk_check_cu_seqlens: bad sizes (nseg %d, total %d)",
               nseg, total);
  check_cu_kernel<<<1, 256, 0, stream>>>(cu, nseg + 1, total, cu_out, status);
  return ditk_check_launch("ditk_check_cu_seqlens");
}

DITK_EXPORT int ditk_patchify(const void* latent, void* out, int C, int F, int H, int W, int pt, int ph,
                              int pw, hipStream_t stream) {
  DITK_REQUIRE(latent && out, "ditk_patchify: null tensor");
  DITK_REQUIRE(pt > 0 && ph > 0 && pw > 0 && F % pt == 0 && H % ph == 0 && W % pw == 0,
               "ditk_patchify: latent %dx%dx%d not divisible by patch %dx%dx%d", F, H, W, pt, ph, pw);
  int64_t n = (int64_t)C * F * H * W;
  patchify_kernel<<<grid_for(n), 256, 0, stream>>>((const bf16_t*)latent, (bf16_t*)out, C, F, H, W, pt, ph, pw);
  return ditk_check_launch("ditk_patchify");
}

DITK_EXPORT int ditk_unpatchify(const void* x, int64_t ldx, float* out, int C, int Fp, int Hp, int Wp,
                                int pt, int ph, int pw, hipStream_t stream) {
  DITK_REQUIRE(x && out, "ditk_unpatchify: null tensor");
  DITK_REQUIRE(ldx >= (int64_t)C * pt * ph * pw, "ditk_unpatchify: ldx too small");
  int64_t n = (int64_t)C * Fp * pt * Hp * ph * Wp * pw;
  unpatchify_kernel<<<grid_for(n), 256, 0, stream>>>((const bf16_t*)x, ldx, out, C, Fp, Hp, Wp, pt, ph, pw);
  return ditk_check_launch("ditk_unpatchify");
}

DITK_EXPORT int ditk_timestep_embedding(const float* t, void* out, int N, int dim, float max_period,
                                        hipStream_t stream) {
  DITK_REQUIRE(t && out && N > 0 && dim > 0 && dim % 2 == 0, "ditk_timestep_embedding: bad arguments");
  int64_t n = (int64_t)N * dim;
  timestep_embed_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(t, (bf16_t*)out, N, dim, logf(max_period));
  return ditk_check_launch("ditk_timestep_embedding");
}

DITK_EXPORT int ditk_cfg_combine(const float* cond, const float* uncond, float* out, int64_t n,
                                 float guidance, hipStream_t stream) {
  DITK_REQUIRE(cond && uncond && out && n >= 0, "ditk_cfg_combine: bad arguments");
  if (n == 0) return 0;
  cfg_combine_kernel<<<grid_for(n), 256, 0, stream>>>(cond, uncond, out, n, guidance);
  return ditk_check_launch("ditk_cfg_combine");
}

DITK_EXPORT int ditk_joint_copy(void* img, int64_t ld_img, void* txt, int64_t ld_txt, void* joint,
                                int64_t ld_joint, const int32_t* cu_img, const int32_t* cu_txt, int nseg,
                                int total, int width, int direction, hipStream_t stream) {
  DITK_REQUIRE(img && txt && joint && cu_img && cu_txt && nseg > 0, "ditk_joint_copy: null argument");
  DITK_REQUIRE(width % 8 == 0 && ld_img % 8 == 0 && ld_txt % 8 == 0 && ld_joint % 8 == 0,
               "ditk_joint_copy: widths must be multiples of 8");
  DITK_REQUIRE(direction == 0 || direction == 1, "ditk_joint_copy: direction must be 0 or 1");
  if (total == 0) return 0;
  joint_copy_kernel<<<total, 64, 0, stream>>>((bf16_t*)img, ld_img, (bf16_t*)txt, ld_txt, (bf16_t*)joint,
                                              ld_joint, cu_img, cu_txt, nseg, total, width, direction);
  return ditk_check_launch("ditk_joint_copy");
}

DITK_EXPORT int ditk_silu(const void* x, void* y, int64_t n, hipStream_t stream) {
  DITK_REQUIRE(x && y && n >= 0, "ditk_silu: bad arguments");
  if (n == 0) return 0;
  silu_kernel<<<grid_for(n), 256, 0, stream>>>((const bf16_t*)x, (bf16_t*)y, n);
  return ditk_check_launch("ditk_silu");
}

DITK_EXPORT int ditk_solver_step(const float* x, const float* cond, const float* uncond, const float* x_last,
                                 const float* m_prev, const float* m_prev2, float* x_next, float* x_corr,
                                 float* m_out, int64_t n, const float* coef, hipStream_t stream) {
  DITK_REQUIRE(x && cond && x_next && coef && n >= 0, "ditk_solver_step: bad arguments");
  SolverCoef k;
  k.g = coef[0]; k.sigma = coef[1]; k.ax = coef[2]; k.a0 = coef[3]; k.a1 = coef[4]; k.a2 = coef[5];
  k.a3 = coef[6]; k.b0 = coef[7]; k.b1 = coef[8]; k.b2 = coef[9]; k.bv = coef[10];
  k.use_uncond = uncond != nullptr;
  k.use_xl = k.a0 != 0.f;
  k.use_mp = k.a1 != 0.f || k.b2 != 0.f;
  k.use_mp2 = k.a2 != 0.f;
  DITK_REQUIRE((!k.use_xl || x_last) && (!k.use_mp || m_prev) && (!k.use_mp2 || m_prev2),
               "ditk_solver_step: a history buffer with a non-zero coefficient is null");
  if (n == 0) return 0;
  solver_step_kernel<<<grid_for(n), 256, 0, stream>>>(x, cond, uncond, x_last, m_prev, m_prev2, x_next, x_corr,
                                                      m_out, n, k);
  return ditk_check_launch("ditk_solver_step");
}
