/*
 * ditk — MI355X (gfx950) kernels for ditserve's per-step DiT transformer forward.
 *
 * C ABI: plain device pointers, sizes and a hipStream_t (passed as void*).
 * Every entry point validates its arguments before launching, launches
 * asynchronously on `stream` (never synchronises), and returns 0 on success or
 * a nonzero status whose message ditk_last_error() holds (per thread).  bf16
 * tensors are uint16 arrays, row-major, with explicit leading dimensions in
 * elements.  cu_seqlens arrays are int32 device arrays [nseg + 1] with
 * cu[0] = 0 (build_cu_seqlens semantics).
 *
 * Reference citations are relative to the zydzydQAQ/ditserve tree.
 */
#ifndef DITK_H
#define DITK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ditk_stream_t; /* hipStream_t */

/* Library version (1). */
int ditk_version(void);

/* Message of the last failed call on this thread. */
const char* ditk_last_error(void);

/*
 * Fused AdaLN:  y = norm(x) [* weight + bias] [* (1 + scale[seg]) + shift[seg]] -> bf16.
 * norm_kind 0 = LayerNorm (biased variance), 1 = RMSNorm; eps inside rsqrt.
 * shift/scale: fp32 per segment, row stride mod_stride (may be NULL: no modulation).
 * weight/bias: fp32 [D] (may be NULL).  In place (y == x) is allowed; x and y
 * may be NULL when T == 0 (nothing is launched).
 * Replaces: Wan AdaLN-1/AdaLN-3 and norm2 — workers/ditserve/models/wan/block.py:283,288,291;
 *   Wan prediction norm_out — block.py:436-446; SD3.5 packed AdaLN-Zero / AdaLN-Continuous —
 *   workers/ditserve/models/sd35_batch.py:336-393; Wan cross-attention norm_q/norm_k
 *   (RMSNorm across heads) — workers/xfuser/model_executor/models/transformers/transformer_wan.py:165-166.
 */
int ditk_adaln(const void* x, int64_t ldx, void* y, int64_t ldy, int T, int D, const int32_t* cu_seqlens,
               int nseg, const float* shift, const float* scale, int64_t mod_stride, const float* weight,
               const float* bias, float eps, int norm_kind, ditk_stream_t stream);

/*
 * Several ditk_adaln calls in one launch (1 to 4 jobs of one norm_kind and one
 * ceil(D / 512)); each job's fields are ditk_adaln's arguments and each row is
 * computed exactly as ditk_adaln computes it (a job with T == 0 gets no
 * workgroups).  The jobs run concurrently: a job's output may be its own x
 * (in place) but must not overlap another job's tensors.  For the short rows
 * of a step that would otherwise cost a launch each (SD3.5's 666 text rows
 * beside its image rows).  No reference counterpart: the reference runs these norms as
 * separate module calls (sd35_batch.py:656-668,683-685,697,704-706).
 */
typedef struct ditk_adaln_job {
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
} ditk_adaln_job;
int ditk_adaln_multi(const ditk_adaln_job* jobs, int njobs, ditk_stream_t stream);

/*
 * mod[s, j] = table[j] + proj[s, j] for kd = k*D contiguous fp32 values per segment.
 * Replaces: _split_temb — workers/ditserve/models/wan/block.py:276-280.
 */
int ditk_modulation(const float* table, const float* proj, float* mod, int nseg, int kd, ditk_stream_t stream);

/*
 * In-place QK RMSNorm (across all heads, or per head when per_head != 0) followed
 * by 3D RoPE on interleaved pairs (optional: rope_cos == NULL skips it).
 * rope tables: fp32 [max_pos][head_dim/2]; pair p rotates with the token's frame
 * position when p < t_pairs, row position when p < t_pairs + h_pairs, else column
 * position; grids: int32 [nseg][3] = (F', H', W') per segment.  q and k may be
 * NULL when T == 0 (nothing is launched); positions past max_pos read the last
 * table row.
 * Replaces: _qk_norm_rope_reference and the fused_qk_norm_rope slot —
 *   transformer_wan.py:24-25,111-115,158-191; SD3.5 per-head norm_q/norm_k —
 *   sd35_batch.py:428-431,438-441.
 */
int ditk_qk_norm_rope(void* q, int64_t ldq, void* k, int64_t ldk, int T, int D, int head_dim, const float* wq,
                      const float* wk, float eps, int per_head, const float* rope_cos, const float* rope_sin,
                      int max_pos, const int32_t* cu_seqlens, const int32_t* grids, int nseg, int t_pairs,
                      int h_pairs, ditk_stream_t stream);

/*
 * The same, out of place: q/k rows are read and the normalized, rotated rows
 * written to q_out/k_out (leading dims ldqo/ldko; may equal q/k).  One pass over
 * the rows, so returning new tensors costs no separate copy.
 * Replaces: the fused_qk_norm_rope slot, which returns new q/k tensors and
 *   leaves its inputs untouched — transformer_wan.py:24-25,111-115.
 */
int ditk_qk_norm_rope_out(const void* q, int64_t ldq, const void* k, int64_t ldk, void* q_out, int64_t ldqo,
                          void* k_out, int64_t ldko, int T, int D, int head_dim, const float* wq, const float* wk,
                          float eps, int per_head, const float* rope_cos, const float* rope_sin, int max_pos,
                          const int32_t* cu_seqlens, const int32_t* grids, int nseg, int t_pairs, int h_pairs,
                          ditk_stream_t stream);

/*
 * Several RoPE-free ditk_qk_norm_rope_out calls in one launch (1 to 4 jobs of
 * one ceil(D / 512) and one grouping: per_head and head_dim); outputs may equal
 * the job's own inputs (in place) but must not overlap another job's tensors.
 * Each row is computed exactly as the single call computes it.  For SD3.5's
 * image and text per-head QK RMSNorms of one block.
 * No reference counterpart: the reference's norm_q / norm_k / norm_added_q /
 * norm_added_k are separate module calls (sd35_batch.py:428-431,438-441).
 */
typedef struct ditk_qk_norm_job {
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
} ditk_qk_norm_job;
int ditk_qk_norm_multi(const ditk_qk_norm_job* jobs, int njobs, ditk_stream_t stream);

/*
 * bf16 MFMA GEMM  C = epilogue(A[M,K] W[N,K]^T + bias[N]) with epilogue
 *   0 bias, 1 GELU-tanh, 2 gated residual R + bf16(y) * gate[seg] (fp32 math),
 *   3 residual R + bf16(y), 4 fp32 output, 5 SiLU.
 * C may alias R.  No split-K: results do not depend on M or on row position.
 * One kernel launch on `stream`, or two when a short last 256-row tile row is
 * left to a small-tile launch (rows are split, never k).
 * K % 32 == 0, N % 8 == 0; A, W, C, R and bias (fp32 [N] or NULL) 16-byte aligned.
 * Replaces: nn.Linear projections of the Wan block (to_q/to_k/to_v/to_out,
 *   ffn.net.0/ffn.net.2) — transformer_wan.py:50-69,154-155; block.py:285,293;
 *   SD3.5 packed GEMMs — sd35_batch.py:411-437,696-708; condition/text embedders.
 */
int ditk_gemm(const void* A, int64_t lda, const void* W, int64_t ldw, const float* bias, void* C, int64_t ldc,
              int M, int N, int K, int epilogue, const void* R, int64_t ldr, const float* gate,
              int64_t gate_stride, const int32_t* cu_seqlens, int nseg, ditk_stream_t stream);

/*
 * Two ditk_gemm products of the same N, K and epilogue, each with its own
 * operands (suffix 0 and 1; arguments as ditk_gemm's), in one launch when the
 * two tile lists together take no more rounds of the GPU's CUs than the larger
 * product alone, give or take 0.4 of a round (else two launches).  Every row
 * equals, bitwise, what ditk_gemm computes for it.  Since the products may run
 * concurrently, C0 must not overlap A1, W1, R1, bias1, gate1 or C1, nor C1 any
 * of product 0's operands; each C may still alias its own R.
 * Replaces: the image- and context-stream projections of one SD3.5 joint block,
 *   issued back to back: attn.to_out / attn.to_add_out (sd35_batch.py:573-579)
 *   and the second linear of ff / ff_context (sd35_batch.py:698,707).
 */
int ditk_gemm_pair(const void* A0, int64_t lda0, const void* W0, int64_t ldw0, const float* bias0, void* C0,
                   int64_t ldc0, int M0, const void* R0, int64_t ldr0, const float* gate0, int64_t gate_stride0,
                   const int32_t* cu_seqlens0, int nseg0, const void* A1, int64_t lda1, const void* W1,
                   int64_t ldw1, const float* bias1, void* C1, int64_t ldc1, int M1, const void* R1, int64_t ldr1,
                   const float* gate1, int64_t gate_stride1, const int32_t* cu_seqlens1, int nseg1, int N, int K,
                   int epilogue, ditk_stream_t stream);

/* Columns of the transposed-V buffer for Tk keys in nseg segments (upper bound). */
int64_t ditk_vt_columns(int64_t Tk, int nseg);

/*
 * V [Tk, ldv] (head h at columns h*head_dim) -> Vt [heads][head_dim][vt_ld] with
 * segment m starting at a 64-aligned column; padding columns are zeroed.
 * Staging for ditk_flash_attn_varlen (no reference counterpart: the layout change
 * that feeds V to the MFMA as a K-contiguous operand).
 */
int ditk_transpose_v(const void* v, int64_t ldv, void* vt, int64_t vt_ld, int Tk, int heads, int head_dim,
                     const int32_t* cu_k, int nseg, ditk_stream_t stream);

/*
 * Varlen block-diagonal flash attention forward (non-causal, no dropout):
 * segment m's queries [cu_q[m], cu_q[m+1]) attend to keys [cu_k[m], cu_k[m+1]).
 * head_dim 64 or 128; out bf16 [Tq, heads*head_dim]; lse (optional, may be NULL)
 * fp32 [heads][lse_ld], natural log of the softmax denominator.  Q and out rows
 * are addressed in 64 bits (a packed Q may span more than 4 GiB); Tq < 2^30,
 * ldk and vt_ld < 2^23.
 * Replaces: the attention backend call Spec.run -> sdpa/aiter kernels —
 *   workers/xfuser/core/attention/spec.py:283-304, backends/sdpa/kernel.py:30-56,
 *   backends/aiter/kernel.py:105-128 (via usp.py:815-824 and usp.py:875-908), and the
 *   SD3.5 varlen slot _FLASH_ATTN_VARLEN_FUNC — sd35_batch.py:19-119,448-486.
 */
int ditk_flash_attn_varlen(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* vt, int64_t vt_ld,
                           void* o, int64_t ldo, float* lse, int64_t lse_ld, const int32_t* cu_q,
                           const int32_t* cu_k, int nseg, int Tq, int heads, int head_dim, float softmax_scale,
                           ditk_stream_t stream);

/*
 * ditk_flash_attn_varlen with q already multiplied by softmax_scale * log2(e)
 * (head_dim 64 or 128).  A producer that folds that factor into its QK-norm
 * weight still rounds q to bf16 once, and the kernel then starts its score
 * accumulators at -max and exponentiates them directly, one fused multiply-add
 * per score fewer.  No reference counterpart: used by the Wan self- and
 * cross-attention (the q RMSNorm weights of transformer_wan.py:50-69 pre-
 * multiplied) and the SD3.5 dual attention, which replaces the reference's SD3.5
 * varlen slot (sd35_batch.py:19-119,448-486) with its per-head RMSNorm weight
 * pre-multiplied.
 */
int ditk_flash_attn_varlen_q_prescaled(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* vt,
                                       int64_t vt_ld, void* o, int64_t ldo, float* lse, int64_t lse_ld,
                                       const int32_t* cu_q, const int32_t* cu_k, int nseg, int Tq, int heads,
                                       int head_dim, ditk_stream_t stream);

/*
 * Joint attention over two packed sources, q pre-scaled as above (head_dim 64).
 * Joint segment m is the rows [cu_a[m], cu_a[m+1]) of the "a" operands followed
 * by the rows [cu_b[m], cu_b[m+1]) of the "b" operands (cu_joint = cu_a + cu_b);
 * each attends to its own joint segment, and o_a / o_b receive the outputs of
 * the a / b rows.  q_a, q_b share ldq; k_a, k_b share ldk; o_a, o_b share ldo.
 * Bitwise equal to gathering the joint rows, ditk_flash_attn_varlen_q_prescaled,
 * and scattering the result.  No reference counterpart: SD3.5's image (a) and
 * text (b) streams enter joint attention without the gather the reference does
 * (sd35_batch.py:230-317) and leave it without the scatter.
 */
int ditk_joint_attn_q_prescaled(const void* q_a, const void* q_b, int64_t ldq, const void* k_a, const void* k_b,
                                int64_t ldk, const void* vt, int64_t vt_ld, void* o_a, void* o_b, int64_t ldo,
                                const int32_t* cu_a, const int32_t* cu_b, const int32_t* cu_joint, int nseg,
                                int T_joint, int heads, int head_dim, ditk_stream_t stream);

/*
 * ditk_transpose_v over the joint rows of two sources (v_a, v_b sharing ldv),
 * laid out as ditk_transpose_v lays out the gathered joint V.  No reference
 * counterpart (staging for ditk_joint_attn_q_prescaled).
 */
int ditk_transpose_v_joint(const void* v_a, const void* v_b, int64_t ldv, void* vt, int64_t vt_ld, int T_joint,
                           int heads, int head_dim, const int32_t* cu_a, const int32_t* cu_b,
                           const int32_t* cu_joint, int nseg, ditk_stream_t stream);

/*
 * latent [C, F, H, W] bf16 -> patches [S, C*pt*ph*pw] bf16 (Conv3d weight order).
 * Replaces: the patch_embedding input gather — transformer_wan.py:328-329.
 */
int ditk_patchify(const void* latent, void* out, int C, int F, int H, int W, int pt, int ph, int pw,
                  ditk_stream_t stream);

/*
 * x [S, pt*ph*pw*C] bf16 -> fp32 latent [C, F'*pt, H'*ph, W'*pw].
 * Replaces: prediction's reshape/permute — transformer_wan.py:391-395, block.py:446-448.
 */
int ditk_unpatchify(const void* x, int64_t ldx, float* out, int C, int Fp, int Hp, int Wp, int pt, int ph, int pw,
                    ditk_stream_t stream);

/*
 * Sinusoidal timestep embedding, bf16 [N, dim], cos half first, frequency shift 0.
 * Replaces: the Timesteps projection inside condition_embedder — transformer_wan.py:331-333.
 */
int ditk_timestep_embedding(const float* t, void* out, int N, int dim, float max_period, ditk_stream_t stream);

/*
 * out = uncond + guidance * (cond - uncond), fp32.
 * Replaces: CFG combine — workers/ditserve/models/wan/block.py:483, runtime.py:689, sd35.py:944.
 */
int ditk_cfg_combine(const float* cond, const float* uncond, float* out, int64_t n, float guidance,
                     ditk_stream_t stream);

/*
 * Joint-sequence copy for SD3.5: direction 0 gathers image and text rows into
 * joint[cu_img[m] + cu_txt[m] + r] (image rows first), 1 scatters back.
 * Replaces: index_copy_/index_select — sd35_batch.py:458-463,476-484.
 */
int ditk_joint_copy(void* img, int64_t ld_img, void* txt, int64_t ld_txt, void* joint, int64_t ld_joint,
                    const int32_t* cu_img, const int32_t* cu_txt, int nseg, int total, int width, int direction,
                    ditk_stream_t stream);

/* y = silu(x), bf16.  Replaces: the SiLU before time_proj / AdaLN linears. */
int ditk_silu(const void* x, void* y, int64_t n, ditk_stream_t stream);

/*
 * A device cu_seqlens table handed in by a caller (int32 [nseg + 1]) checked on
 * the GPU and made safe before a segment kernel reads it: cu_out[0] = 0 and
 * cu_out[i] = the running max of cu[0..i] clamped into [0, total], so every row
 * the kernels derive from cu_out exists.  A valid table (cu[0] = 0,
 * nondecreasing, cu[nseg] = total) is copied unchanged; any other sets bit 0 of
 * *status, which the kernel never clears (the host reads it after a later sync).
 * No host synchronisation; cu_out must not be cu.
 * Replaces: the trust the reference's varlen slot places in its device tables
 *   (sd35_batch.py:448-486 passes cu_seqlens straight to the flash kernel).
 */
int ditk_check_cu_seqlens(const int32_t* cu, int nseg, int total, int32_t* cu_out, int32_t* status,
                          ditk_stream_t stream);

/*
 * Fused CFG combine + solver step for one request's fp32 latent of n elements,
 * with the step's scalar coefficients coef[11] = {g, sigma, ax, a0, a1, a2, a3,
 * b0, b1, b2, bv} computed on the host:
 *   v  = uncond ? u + g (c - u) : c;   m = x - sigma v
 *   x_corr = ax x + a0 x_last + a1 m_prev + a2 m_prev2 + a3 m
 *   x_next = b0 x_corr + b1 m + b2 m_prev + bv v
 * (UniPC predictor/corrector on flow sigmas, or FlowMatch-Euler with ax = b0 = 1,
 * bv = sigma_next - sigma.)  History pointers may be null where their
 * coefficients are zero; x_corr / m_out may be null (not written).  x_next may
 * alias x, x_corr may alias x_last, m_out may alias m_prev2.
 * Replaces: CFG combine + scheduler.step — workers/ditserve/models/wan/block.py:465-483,
 *   workers/ditserve/models/wan/runtime.py:686-701, workers/ditserve/models/sd35.py:942-953.
 */
int ditk_solver_step(const float* x, const float* cond, const float* uncond, const float* x_last,
                     const float* m_prev, const float* m_prev2, float* x_next, float* x_corr, float* m_out,
                     int64_t n, const float* coef, ditk_stream_t stream);

/* Size of the per-GPU scratch array behind ditk_flash_attn_varlen_noalloc (64 MiB). */
#define DITK_NOALLOC_SCRATCH_BYTES (64u << 20)

/*
 * ditk_flash_attn_varlen that allocates nothing: V is taken row-major
 * ([Tk, ldv], head h at columns h*head_dim, as ditk_transpose_v takes it) and
 * transposed into a file-scope device array of DITK_NOALLOC_SCRATCH_BYTES that
 * each GPU holds until the process ends, then attended exactly as by
 * ditk_transpose_v + ditk_flash_attn_varlen (bitwise the same outputs and lse).
 * Calls needing more than the scratch (heads * head_dim * ditk_vt_columns(Tk,
 * nseg) * 2 bytes) are rejected before any launch.  Every call on a GPU shares
 * that GPU's array: calls that overlap on one GPU (on different streams) race.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 */
int ditk_flash_attn_varlen_noalloc(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                                   void* o, int64_t ldo, float* lse, int64_t lse_ld, const int32_t* cu_q,
                                   const int32_t* cu_k, int nseg, int Tq, int Tk, int heads, int head_dim,
                                   float softmax_scale, ditk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DITK_H */
