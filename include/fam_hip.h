/*
 * fam_hip.h -- C ABI of the MI355X (gfx950) kernels for the FastWAM / DiT4DiT
 * action-DiT denoising hot path.
 *
 * Every entry point takes plain device pointers, element counts and strides, and
 * the HIP stream to launch on (a hipStream_t passed as void*; NULL = the null
 * stream).  The library never allocates and uses no scratch memory: the caller owns
 * every buffer, so every entry point can be recorded into a HIP graph.
 * Tensors are bf16 unless a parameter says fp32.  Strides are in elements.
 *
 * Return value: FAM_OK, or an error code with a message readable through
 * fam_last_error() (thread-local).  Argument validation happens before any launch,
 * so an error return means nothing was enqueued.
 *
 * Reference paths below are relative to the reference checkout:
 *   FB  = src/fastwam-baseline/fastwam/models/wan22
 *   FG  = src/fastwam-geak/fastwam/models/wan22
 *   CA  = src/cae-fastwam/fastwam/models/wan22
 *   SCH = FB/schedulers/scheduler_continuous.py
 */
#ifndef FAM_HIP_H
#define FAM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FAM_OK 0
#define FAM_ERR_INVALID_ARG 1
#define FAM_ERR_UNSUPPORTED 2
#define FAM_ERR_LAUNCH 3

#define FAM_ABI_VERSION 3

/*
 * No entry point allocates, keeps state between calls or communicates between
 * workgroups: every launch is self-contained, deterministic (fixed reduction order, no
 * float atomics) and may be recorded into a HIP graph.
 */

/* Library ABI version (FAM_ABI_VERSION). */
int fam_version(void);

/* Message of the last error returned on this thread ("" if none). */
const char* fam_last_error(void);

/*
 * fam_set_launch_events -- profiling aid with no counterpart in the reference: after a pair
 * of hipEvent_t (created with timing enabled) is armed on the calling thread, the first kernel
 * the library launches records start_event at its begin and every kernel records stop_event at
 * its end (hipExtLaunchKernelGGL), so hipEventElapsedTime spans the kernels of one call (a
 * call such as fam_gemm_ws launches two); arm a fresh pair per call.  Pass two nulls to
 * disarm.  Not for use under stream capture.
 */
int fam_set_launch_events(void* start_event, void* stop_event);

/*
 * fam_adaln -- LayerNorm over the last dim with AdaLN-Zero modulation:
 *   y[r,:] = (LN(x[r,:]) [* ln_weight + ln_bias]) * (1 + scale[r,:]) + shift[r,:]
 * LN is biased-variance, eps inside the rsqrt, fp32 statistics.
 * shift/scale (both or neither) are indexed as
 *   base + (r / rows_per_batch) * mod_batch_stride + (r % rows_per_batch) * mod_row_stride
 * so mod_row_stride = 0 broadcasts one vector over a batch's tokens ([B,1,D]) and
 * mod_row_stride = D gives per-token modulation ([B,S,D]).  ln_weight / ln_bias may be
 * NULL (elementwise_affine=False).
 * Replaces: adaln_forward(x, norm, shift, scale)   FB/fused_adaln.py:513-523
 *           (eager branch :522-523; used FB/wan_video_dit.py:281,284, FB/mot.py:125,169),
 *           DiTBlock.norm3                          FB/wan_video_dit.py:261,283,
 *           modulate(norm(x), shift, scale)         CA/wan_video_dit.py:590-591.
 * Limits: dim % 8 == 0, 8 <= dim <= 16384; x/y rows 16-byte aligned.
 */
int fam_adaln(const void* x, int64_t x_row_stride,
              const void* shift, const void* scale,
              int64_t mod_batch_stride, int64_t mod_row_stride,
              const void* ln_weight, const void* ln_bias,
              void* y, int64_t y_row_stride,
              int64_t rows, int64_t rows_per_batch, int64_t dim, float eps, void* stream);

/*
 * fam_rmsnorm_rope -- RMSNorm then rotary embedding, per row:
 *   n = bf16(x * rsqrt(mean(x^2) + eps)) * weight          (skipped if weight == NULL)
 *   y[2i], y[2i+1] = n[2i] c - n[2i+1] s,  n[2i] s + n[2i+1] c   (skipped if cos_tab == NULL)
 * with (c, s) = (cos_tab, sin_tab)[pos * tab_row_stride + j * tab_elem_stride], pos = row % seq_len,
 * j = pair index within the head (0 .. head_dim/2-1).  Tables are fp32.  The RMS is over the
 * full row (all heads), as RMSNorm(H*Dh) in the reference.  y may equal x (in place).
 * Replaces: RMSNorm.forward                 FB/wan_video_dit.py:156-167,
 *           rope_apply(x, freqs, num_heads) FB/wan_video_dit.py:58-70, FG/wan_video_dit.py:193-215,
 *                                           CA/wan_video_dit.py:769-799,
 *           fused q/k post-processing       FG/mot.py:786-816 (qkv_post without the K/V cache write).
 * Limits: dim % 8 == 0, dim <= 16384, head_dim even and dim % head_dim == 0 (rope);
 * 16-byte aligned rows.
 */
int fam_rmsnorm_rope(const void* x, int64_t x_row_stride, void* y, int64_t y_row_stride,
                     int64_t rows, int64_t seq_len, int64_t dim,
                     const void* weight, float eps,
                     const float* cos_tab, const float* sin_tab,
                     int64_t tab_row_stride, int64_t tab_elem_stride, int64_t head_dim,
                     void* stream);

/*
 * fam_rmsnorm_grouped -- RMSNorm of every row with one of `groups` weight vectors:
 *   y[r] = bf16(x[r] * rsqrt(mean(x[r]^2) + eps)) * weights[(r % groups) * dim ..]
 * with the rounding of fam_rmsnorm_rope.  One launch for the context keys of every block of
 * a prefill: rows = (context rows) x (blocks), row stride = the stride between consecutive
 * blocks' keys, group = block.
 * Replaces: RMSNorm.forward of each block's cross_attn.norm_k (FB/wan_video_dit.py:156-167,
 *           applied per block at FB/wan_video_dit.py:226).
 * Limits: as fam_rmsnorm_rope; rows % groups == 0; weights [groups, dim] 16-byte aligned.
 */
int fam_rmsnorm_grouped(const void* x, int64_t x_row_stride, void* y, int64_t y_row_stride,
                        int64_t rows, int64_t dim, const void* weights, int64_t groups, float eps,
                        void* stream);

/*
 * fam_headnorm_rope -- per-head RMSNorm, then rotate-half RoPE, over nseg column segments of
 * each row (the Cosmos backbone's q / k).  Segment s covers columns [s * seg_stride,
 * s * seg_stride + width) in heads of head_dim; for each head h of row r:
 *   n = bf16(bf16(x_h * rsqrt(mean(x_h^2) + eps)) * weight[s * weight_seg_stride + d])
 *   rope (cos_tab != NULL): y_h[d] = bf16(n[d] c[d] + r[d] s[d]),  r = cat(-n[D/2:], n[:D/2]),
 *     (c, s) = (cos_tab, sin_tab)[(r % seq_len) * tab_row_stride + d], fp32 tables [S, head_dim]
 *     whose halves repeat the same angles (pairs (d, d + head_dim / 2))
 * y may equal x.  One launch normalises q and k of a block (nseg = 2, seg_stride = A, weights
 * [norm_q; norm_k]) or the context keys of every block (nseg = blocks).
 * Replaces: CosmosAttnProcessor2_0's norm_q / norm_k (RMSNorm(attention_head_dim), diffusers'
 *           RMSNorm: bf16 rounding before the weight) and apply_rotary_emb(use_real=True,
 *           use_real_unbind_dim=-2) (src/dit4dit-geak/patches/diffusers-3996788-transformer_cosmos-
 *           geak.patch:1289-1316, 1525-1710; the fused form _geak_qkrope :846-907).
 * Limits: head_dim a power of two in [16, 512]; width a multiple of head_dim; strides and
 * seg_stride multiples of 8 elements; 16-byte aligned x, y, weight and tables.
 */
int fam_headnorm_rope(const void* x, int64_t x_row_stride, void* y, int64_t y_row_stride, int64_t rows,
                      int64_t seq_len, int64_t nseg, int64_t seg_stride, int64_t width, int64_t head_dim,
                      const void* weight, int64_t weight_seg_stride, float eps, const float* cos_tab,
                      const float* sin_tab, int64_t tab_row_stride, void* stream);

/*
 * fam_act_rows -- y[r, c] = bf16(act(x[r, c])) for rows x cols (act FAM_ACT_*).
 * Replaces: the SiLU of CosmosAdaLayerNormZero.forward (`self.activation(embedded_timestep)`,
 *           shared by every AdaLN unit of the Cosmos blocks; the patch applies it once,
 *           diffusers-3996788-transformer_cosmos-geak.patch:2171-2175).
 * Limits: cols and row strides multiples of 8; 16-byte aligned rows.
 */
int fam_act_rows(const void* x, int64_t x_row_stride, void* y, int64_t y_row_stride, int64_t rows, int64_t cols,
                 int act, void* stream);

/* Attention mask kinds for fam_attn_desc.mask_kind. */
#define FAM_MASK_NONE 0
#define FAM_MASK_BOOL 1      /* uint8, nonzero = attend (torch bool)      */
#define FAM_MASK_ADD_F32 2   /* fp32 added to the scaled scores           */
#define FAM_MASK_ADD_BF16 3  /* bf16 added to the scaled scores           */

/*
 * Attention over [B, H] heads: o = softmax(q k^T * scale + mask) v, fp32 softmax.
 * Element (b, s, h, d) of tensor t lives at t + b*t_bs + s*t_rs + h*t_hs + d, which covers
 * both [B,S,H*Dh] (t_hs = Dh) and [B,H,S,Dh] (t_rs = Dh, t_hs = S*Dh) layouts.  The keys and
 * values are the concatenation of two segments: keys 0..sk0-1 from (k0, v0) and
 * sk0..sk0+sk1-1 from (k1, v1) (sk1 = 0: one segment), e.g. a cached video prefix followed
 * by the action tokens.  The mask element for (b, h, q, key) is
 * mask[b*mask_bs + h*mask_hs + q*mask_qs + key].  A query row with every key masked gives 0.
 * Work split (head_dim 64 / 128): up to 32 queries over their own <= 32 unmasked keys, one
 * workgroup per (b, h) with q, k and v staged in LDS; up to 32 queries over <= 256 keys (up to
 * 128 queries when q is not normalised on load, as chunks of 32), one workgroup per (b, h) and
 * chunk whose waves split the keys (partial softmax states merged in LDS in a fixed order); up
 * to 32 queries over one long unmasked key segment, one workgroup per (b, h) and key split;
 * longer query sequences over one key segment with no mask or a key-only boolean mask, 128
 * queries per workgroup with the K/V tiles streamed through LDS (at head_dim 128 on a grid of
 * at most one workgroup per CU, two groups of waves take alternate tiles and merge in LDS);
 * otherwise (and for the other head dims) one workgroup per (b, h) holding all queries up to
 * 32 (64 for head_dim < 128), 64 queries per workgroup beyond.  Every path gives the same result up to fp32 summation
 * order; for a given shape and arguments the path, and so the bits, are fixed.
 * Replaces: flash_attention(q, k, v, num_heads, ctx_mask)  FB/wan_video_dit.py:17-26,
 *           FG/wan_video_dit.py:18-39, CA/wan_video_dit.py:569-587;
 *           fastwam::short_attn / short_attn_bsd          FG/wan_video_dit.py:1680-1721, FG/mot.py:682-722;
 *           joint [video cache; action] attention          FB/mot.py:446-478.
 * Limits: head_dim in {8, 16, 32, 64, 128}; all strides multiples of 8; 16-byte aligned
 * bases; batch*heads <= 65535 when Sq > 64.
 */
typedef struct fam_attn_desc {
  const void* q;  int64_t q_bs, q_rs, q_hs;
  const void* k0; int64_t k0_bs, k0_rs, k0_hs;
  const void* v0; int64_t v0_bs, v0_rs, v0_hs;
  const void* k1; int64_t k1_bs, k1_rs, k1_hs;
  const void* v1; int64_t v1_bs, v1_rs, v1_hs;
  void* o;        int64_t o_bs, o_rs, o_hs;
  int64_t batch, heads, sq, sk0, sk1, head_dim;
  float scale;
  const void* mask; int mask_kind; int64_t mask_bs, mask_hs, mask_qs;
  int num_splits; float* part_o; float* part_ml;
  /* RMSNorm (+ RoPE) of q and/or k applied as they are loaded (qk_norm = 1); see below. */
  int qk_norm;
  const float* q_sumsq; const float* k_sumsq;
  int64_t ss_row_stride, ss_batch_rows, q_group0, k_group0, norm_width;
  const void* q_norm_w; const void* k_norm_w;
  float norm_eps;
  const float* rope_cos; const float* rope_sin; int64_t rope_row_stride;
} fam_attn_desc;

int fam_attention(const fam_attn_desc* d, void* stream);

/*
 * On-load q/k normalisation (qk_norm = 1, short-query path only): q and k arrive as the raw
 * projections (fam_gemm_final output, bias added) and are normalised the way the reference's
 * q/k post-processing does, RMSNorm over the full H*Dh row with a bf16 rounding before the
 * weight, then the RoPE rotation of (d, d+1) pairs (FB/wan_video_dit.py:156-167, 58-70,
 * 193-196, 215-216):
 *   rstd(b, s) = rsqrt(sum_{g < norm_width/16} ss[row*ss_row_stride + group0 + g] / norm_width + eps),
 *   row = b*ss_batch_rows + s, ss = q_sumsq / k_sumsq (fam_gemm_final's sums of squares);
 *   y[d] = bf16(bf16(x[d] * rstd) * w[h*head_dim + d]);
 *   with rope_cos/sin (complex layout [pos][head_dim/2], row stride rope_row_stride, pos = s):
 *   (y[2j], y[2j+1]) rotated by (cos, sin)[s][ (d of y[2j]) / 2 ].
 * A null q_sumsq / k_sumsq leaves that side as loaded.
 * Limits: head_dim 64 or 128; norm_width a multiple of 1024; ss_row_stride, q_group0, k_group0
 * and rope_row_stride multiples of 4; one key segment when k is normalised; 16-byte aligned
 * weights and tables.
 */

/*
 * Key split over workgroups (Sq <= 32, or <= 64 for head_dim < 128): with num_splits = S > 1,
 * fam_attention writes, instead of o, the unnormalised partial output of each split to
 * part_o [S][B*H][Sq][head_dim] (fp32) and its (running max in log2 units, sum) to
 * part_ml [S][B*H][Sq][2]; fam_attention_combine then merges the splits in order into o.
 * The caller allocates both buffers.  Two launches, no cross-workgroup synchronisation.
 */
int fam_attention_combine(const fam_attn_desc* d, void* stream);

/*
 * fam_attention_key_splits -- the num_splits to use for an unmasked, single-segment attention
 * of sq queries over sk keys: the cross-attention over the context (replaces the split choice
 * around flash_attention in CrossAttention.forward, FB/wan_video_dit.py:224-229).  Returns 1
 * up to 256 keys (one workgroup per head takes every key), otherwise about four 32-key blocks
 * per split (one per wave of the split's workgroup), at most 64.  Each split's workgroup runs
 * its own softmax, so the splits spread that vector work over the CUs; splitting a head's
 * output dims instead (every workgroup scoring every key) multiplied it and measured slower.
 * A deterministic function of the shape; 0 for invalid arguments.
 */
int fam_attention_key_splits(int64_t batch, int64_t heads, int64_t sq, int64_t sk, int64_t head_dim);

/*
 * fam_attention_noalloc -- fam_attention with key splits followed by fam_attention_combine,
 * with the split partials in a library-owned device array (8 MiB per GPU, held until the
 * process ends) instead of the caller's part_o / part_ml, which are ignored.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc); it calls no allocating
 * routine.  The caller passes q, k, v and o as for fam_attention; num_splits in [2, 64] and
 *   num_splits * batch * heads * sq * (head_dim + 2) * 4 bytes <= fam_attention_noalloc_max_bytes()
 * (larger calls return FAM_ERR_UNSUPPORTED).  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams, or host threads) race and must be
 * serialised by the caller.  Results equal fam_attention + fam_attention_combine bit for bit.
 * fam_attention_noalloc_max_bytes is the set-up call: made once per device with that device
 * current (before any graph capture), it looks up the array's device address and returns the
 * scratch size, or -FAM_ERR_LAUNCH when the lookup fails; a device whose set-up call was never
 * made is set up by its first fam_attention_noalloc.
 */
int fam_attention_noalloc(const fam_attn_desc* d, void* stream);
int64_t fam_attention_noalloc_max_bytes(void);

/* GEMM prologues (applied to each row of A before the product) and activations. */
#define FAM_PRO_NONE 0
#define FAM_PRO_LAYERNORM 1  /* LN(a) [* pro_w + pro_b]                        */
#define FAM_PRO_ADALN 2      /* LN(a) * (1 + pro_scale) + pro_shift            */
#define FAM_PRO_LN_FOLDED 3  /* LN(a) with its affine / modulation folded into w, bias (below) */
#define FAM_ACT_NONE 0
#define FAM_ACT_GELU_TANH 1
#define FAM_ACT_SILU 2
#define FAM_ACT_RELU 3   /* the DiT4DiT head's MLPs: DB/modules/action_model/ActionDiT.py:52-61 */
#define FAM_ACT_GELU_ERF 4  /* exact GELU, the Cosmos backbone's FeedForward ("gelu"); erff */

/*
 * fam_gemm -- out[m, n] = epilogue( sum_k pro(a)[m, k] * w[n, k] + bias[n] ),
 * w in nn.Linear layout [N, K].  Epilogue, in order: activation; then, if res != NULL,
 * out = res[m, n] + g(m, n) * value with g = 1 when gate == NULL, else
 * g = gate[(m / rows_per_batch) * gate_bs + (m % rows_per_batch) * gate_rs + n * gate_ns]
 * (gate_ns = 0 with gate_bs = gate_rs = 0 makes it one scalar, e.g. the Euler delta).
 * res may equal out (in-place residual update).  out_f32 != 0 makes out and res fp32
 * (e.g. the fused Euler update of fp32 latents); otherwise both are bf16.  AdaLN shift/scale use the same
 * (rows_per_batch, pro_mod_bs, pro_mod_rs) indexing with a unit column stride.
 * FAM_PRO_LN_FOLDED (M <= 64): sum_k LN(a)[m, k] * w[n, k] is evaluated as
 *   rstd_m * (sum_k a[m, k] * w[n, k] - mean_m * pro_w[n]),
 * mean_m and rstd_m = 1/sqrt(var_m + pro_eps) of row m of a over K, pro_w an fp32 [N] vector
 * holding sum_k w[n, k] of the bf16 w; the product runs on the raw rows, so no normalisation
 * sits between the loads and the matrix cores.  A LayerNorm affine (g, b) and an AdaLN
 * modulation (1 + s, t) that are the same for every row fold into w' = w diag(g (1 + s)),
 * bias' = bias + w (b (1 + s) + t) beforehand (fam.ops.fold_layernorm).
 * Work split: for M <= 64 a workgroup of 8 waves owns 16 output columns and the waves split
 * K (reduced through LDS in wave order); for M >= 128 without a prologue and with K % 64 == 0,
 * output tiles of 256x256, 224x256, 128x128, 128x96 or 64x64 chosen for the shape and the
 * device's CU count (128x128 tiles on a grid of at most one workgroup per CU split K between
 * two groups of waves whose sums meet in LDS in a fixed order); otherwise 64x64 or 128x128
 * tiles.  The choice, and so the bits, are a fixed function of the shape on a given device.
 * Replaces: nn.Linear / F.linear on the hot path (FB/wan_video_dit.py:188-191,215-218,262-263,
 *           FB/action_dit.py:76-97,317-318), fastwam::skmm + skpost (split-K GEMM with
 *           bias/gate/residual/norm epilogue, FG/mot.py:1080-1348), geak_head::mmx with the
 *           fused Euler epilogue (DG/modules/action_model/ActionDiT.py:1260-1272).
 * Limits: K % 8 == 0; a, w rows 16-byte aligned (lda, ldw multiples of 8); N <= 1048560.
 */
typedef struct fam_gemm_desc {
  const void* a; int64_t lda;
  const void* w; int64_t ldw;
  const void* bias;
  void* out; int64_t ldo;
  int64_t M, N, K;
  int prologue;
  const void* pro_w; const void* pro_b;
  const void* pro_shift; const void* pro_scale;
  int64_t pro_mod_bs, pro_mod_rs;
  float pro_eps;
  int act;
  const void* res; int64_t ldr;
  const void* gate; int64_t gate_bs, gate_rs, gate_ns;
  int64_t rows_per_batch;
  int out_f32;
} fam_gemm_desc;

int fam_gemm(const fam_gemm_desc* d, void* stream);

/*
 * fam_gemm_ws -- fam_gemm with a caller-owned fp32 workspace: a product inside the large-M
 * kernel's envelope (no prologue, M >= 128, K % 64 == 0, N % 4 == 0) whose tiles cannot fill the
 * GPU (few rows and columns, long K: the deep levels of the VAE encoder) is split along K over
 * workgroups into fp32 planes ws[z][M][N] and finished by fam_rowop (planes summed in split order,
 * then the same bias / activation / gate / residual epilogue); otherwise, or when the workspace
 * is too small for two planes, it is exactly fam_gemm.  fam_gemm_ws_floats(M, N, K) is the
 * workspace (floats) of the split the plan picks for the shape when the workspace does not
 * limit it, splits * M * N (0: the plan does not split); a smaller workspace limits the split.
 * Replaces: as fam_gemm; the reference's convolutions run here as such GEMMs
 *           (CausalConv3d FB/wan_video_vae.py:33-52 on the first frame).
 * Limits: as fam_gemm; ws 16-byte aligned.
 */
int fam_gemm_ws(const fam_gemm_desc* d, float* ws, int64_t ws_floats, void* stream);
int64_t fam_gemm_ws_floats(int64_t M, int64_t N, int64_t K);

/*
 * fam_gemm_partial -- split-K product without any cross-workgroup traffic:
 * partials[z][m][n] = sum over k in split z of a[m, k] * w[n, k], fp32,
 * z < fam_gemm_partial_splits(M, N, K) (a deterministic function of the shape).  The caller
 * allocates splits*M*N floats and sums them with fam_rowop, which also applies the
 * epilogue.  a [M, K] and w [N, K] bf16 (nn.Linear layout).  Up to 144 rows the weights stream
 * through the small-M kernels; above, the large-M tile kernel writes the planes, split along K
 * only where the extra planes (read by the row kernel that follows anyway) cost less than the
 * idle CUs of an unsplit grid (one plane: the plain fp32 product).
 * Replaces: the projections of the action tokens (q/k/v/o, cross q/o, FFN up/down, head;
 *           FB/wan_video_dit.py:188-191,215-218,262-263, FB/action_dit.py:317-318) and the
 *           reference's split-K kernel fastwam::skmm (FG/mot.py:1080-1243).
 * Limits: M <= 128, or up to 144 where fam_gemm_partial_splits is non-zero (the streaming
 * plan: >= 3 chunks of 256 along K per split, e.g. a prefill's 129-row context K/V of every
 * block), or above 144 with N % 4 == 0, K % 64 == 0, K >= 128 and (M + 256) * lda * 2,
 * (N + 256) * ldw * 2 < 2^31 bytes (fam_gemm_partial_splits returns 0 for an unsupported shape);
 * K % 8 == 0; lda, ldw multiples of 8; 16-byte aligned a, w, partials; from 65 to 144 rows
 * lda, ldw < 2^23 elements.
 */
int fam_gemm_partial(const void* a, int64_t lda, const void* w, int64_t ldw, float* partials,
                     int64_t M, int64_t N, int64_t K, void* stream);
int fam_gemm_partial_splits(int64_t M, int64_t N, int64_t K);

/*
 * fam_gemm_final -- out[m, n] = bf16(act(sum_k a[m, k] * w[n, k] + bias[n])) for 1 <= M <= 64
 * with the whole K of 16 output columns in one workgroup (no partials, no second kernel).
 * If sumsq is non-null it also receives, for every row m and 16-column group g < G = ceil(N/16),
 *   sumsq[m * G + g] = sum over the group's columns of out[m, n]^2   (of the stored bf16 values),
 * the statistics a later RMSNorm over any union of whole groups needs (fam_attention's q/k
 * normalisation).  a [M, K], w [N, K] bf16; bias bf16 [N] or null; act FAM_ACT_*.
 * Replaces: the q/k/v, cross-q and FFN-up projections of the action tokens
 *           (FB/wan_video_dit.py:188-191, 215, 262) with their bias/GELU epilogues.
 * Limits: M <= 64; K % 8 == 0, K <= 4096; lda, ldw multiples of 8; a, w 16-byte and out
 *         8-byte aligned; sumsq holds M*ceil(N/16) floats.
 */
int fam_gemm_final(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias, int act,
                   void* out, int64_t ldo, float* sumsq, int64_t M, int64_t N, int64_t K, void* stream);

/* Row sources and row normalisations for fam_rowop. */
#define FAM_ROWSRC_PARTIALS 0   /* sum of fam_gemm_partial splits                 */
#define FAM_ROWSRC_SMALLK 1     /* x_in [M, k_in] fp32 times w_in [N, k_in] bf16  */
#define FAM_ROWNORM_NONE 0
#define FAM_ROWNORM_LAYERNORM 1 /* LN(row) [* ln_weight + ln_bias]                */
#define FAM_ROWNORM_ADALN 2     /* LN(row) * (1 + scale) + shift                  */
#define FAM_ROWNORM_RMS 3       /* RMSNorm (+ RoPE) of 1 or 2 column segments     */

/*
 * fam_rowop -- one workgroup per row m < M of width N:
 *   v = source(m, n) + bias[n];  v = act(v);
 *   if res: v = res[m, n] + g(m, n) * v  (g as in fam_gemm: gate[(m/rpb)*gate_bs +
 *           (m%rpb)*gate_rs + n*gate_ns], 1 without a gate);
 *   out[m, n] = v  (bf16, or fp32 with res when out_f32);
 *   then, on the stored row:
 *     LAYERNORM  nout = LN(v) [* ln_weight + ln_bias]
 *     ADALN      nout = LN(v) * (1 + scale) + shift, modulation indexed like fam_adaln
 *     RMS        for each segment g < nseg: columns [seg_col0[g], seg_col0[g] + seg_width):
 *                nout = rope(bf16(bf16(v * rsqrt(mean(v^2) + eps)) * seg_weight[g][col])),
 *                rope as in fam_rmsnorm_rope (skipped when rope_cos == NULL; position =
 *                m % seq_len); other columns of nout are not written (nout may equal out).
 * LN statistics are biased-variance, eps inside the rsqrt, fp32, reduced in a fixed order.
 * Replaces the epilogues and the norms between the reference's projections:
 *   gate/residual  FB/wan_video_dit.py:232-237,282-285;  adaln_forward FB/fused_adaln.py:513-523;
 *   norm3          FB/wan_video_dit.py:261,283;  RMSNorm + rope_apply FB/wan_video_dit.py:156-167,58-70;
 *   GELU           FB/wan_video_dit.py:262;  the reference's fused epilogue kernels fastwam::skpost,
 *   qkv_post, res_ln* (FG/mot.py:1280-1348, 786-816, 1771-1941); the Euler update of
 *   geak_head::mmx (DG/modules/action_model/ActionDiT.py:1260-1272) with out_f32.
 * Partials source: v = sum over z < splits of partials[z * split_stride + m * ldp + n] (ldp = N when
 * 0): with ldp above N a row kernel reads a column window of wider planes (a q/k/v split-K
 * product finished segment by segment).
 * Limits: 1 <= N <= 4096, or any N < 2^30 when the row is vectorisable (partials source,
 * N % 4 == 0, <= 64 splits, ldo / ldp / ldr multiples of 4, 8-byte aligned bf16 operands,
 * 16-byte aligned fp32 ones) and either has no normalisation or RMS segments that each fill
 * one tile (seg_width in {1024, 2048, 3072, 4096}, seg_col0 multiples of seg_width: a
 * q | k | v row); a normalised row must be bf16 (out_f32 == 0).
 */
typedef struct fam_rowop_desc {
  int src;
  const float* partials; int64_t splits, split_stride;
  const float* x_in; int64_t ldx, k_in; const void* w_in;
  int64_t M, N;
  const void* bias; int act;
  const void* res; int64_t ldr;
  const void* gate; int64_t gate_bs, gate_rs, gate_ns; int64_t rows_per_batch;
  void* out; int64_t ldo; int out_f32;
  int norm; float eps;
  const void* ln_weight; const void* ln_bias;
  const void* shift; const void* scale; int64_t mod_bs, mod_rs;
  int nseg; int64_t seg_col0[2]; int64_t seg_width; const void* seg_weight[2];
  const float* rope_cos; const float* rope_sin; int64_t rope_row_stride, rope_elem_stride, head_dim, seq_len;
  void* nout; int64_t ldn;
  int64_t ldp;   /* row stride of the partial planes (elements); 0 means N */
} fam_rowop_desc;

int fam_rowop(const fam_rowop_desc* d, void* stream);

/*
 * fam_linear_smallk -- y[m, n] = sum_k x[m, k] w[n, k] + b[n] for small, unaligned K
 * (the 7-wide action encoder, FB/action_dit.py:76, :285).  x is bf16, or fp32 when
 * x_f32 != 0; w, b and y are bf16; fp32 accumulation.  Limits: K <= 64.
 */
int fam_linear_smallk(const void* x, int64_t ldx, int x_f32, const void* w, const void* b,
                      void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* stream);

/*
 * fam_euler_step -- out[i] = bf16(sample[i] + bf16(model_output[i] * delta[i / inner])), the
 * flow-matching update in the rounding order of the eager bf16 expression
 * `sample + model_output * delta` (SCH:82-88).  delta holds bf16 values in device memory:
 * one scalar (inner = n) or one per batch row ([B] deltas viewed [B,1,...], inner = n / B).
 * n elements, contiguous; out may equal sample (in place).
 * Replaces: WanContinuousFlowMatchScheduler.step  SCH:82-88;
 *           actions - dt * v                       DB/modules/action_model/ActionDiT.py:368.
 */
int fam_euler_step(const void* sample, const void* model_output, const void* delta, void* out,
                   int64_t n, int64_t inner, void* stream);

/*
 * fam_sinusoid -- out[t, :] = bf16(cat(cos(p_t f), sin(p_t f))), f_i = 10000^(-i/(dim/2)),
 * computed in fp64 from the bf16 positions p (FB/wan_video_dit.py:34-38).  out [T, dim].
 */
int fam_sinusoid(const void* positions, void* out, int64_t T, int64_t dim, void* stream);

/*
 * fam_patchify -- the patch gather in front of the patch-embedding GEMM: x [B, C, F, H, W]
 * (contiguous bf16) into rows out[b*S + (fi*h + hi)*w + wi, ((c*pt + kt)*ph + kh)*pw + kw] =
 * x[b, c, fi*pt + kt, hi*ph + kh, wi*pw + kw], S = f*h*w tokens (f = F/pt, h = H/ph, w = W/pw),
 * so that rows x conv_weight.reshape(hidden, -1)^T + bias is the strided Conv3d.
 * Replaces: WanVideoDiT.patchify (nn.Conv3d(in_dim, dim, kernel = stride = patch_size))
 *           FB/wan_video_dit.py:385-386, 420-426.
 * Limits: F, H, W divisible by the patch; B*C*F*H*W < 2^38.
 */
int fam_patchify(const void* x, int64_t B, int64_t C, int64_t F, int64_t H, int64_t W, int64_t pt, int64_t ph,
                 int64_t pw, void* out, void* stream);

/*
 * fam_unpatchify -- the inverse layout after the head GEMM: y [B*S, pt*ph*pw*C] with the
 * features ordered (kt, kh, kw, c) into out [B, C, f*pt, h*ph, w*pw] (contiguous bf16),
 * rearrange 'b (f h w) (x y z c) -> b c (f x) (h y) (w z)'.
 * Replaces: WanVideoDiT.unpatchify FB/wan_video_dit.py:428-433.
 */
int fam_unpatchify(const void* y, int64_t B, int64_t C, int64_t f, int64_t h, int64_t w, int64_t pt, int64_t ph,
                   int64_t pw, void* out, void* stream);

/*
 * fam_gather_rows -- dst[r, :] = src[idx[r], :] for r < rows, cols bf16 elements per row;
 * idx int32 in device memory, clamped into [0, src_rows).  Broadcasts the time embedding and
 * t_mod of the few distinct per-frame timesteps to every token.
 * Replaces: the per-token time_embedding / time_projection rows of WanVideoDiT.pre_dit
 *           (FB/wan_video_dit.py:555-568), computed once per distinct timestep.
 * Limits: cols % 8 == 0; strides multiples of 8; 16-byte aligned.
 */
int fam_gather_rows(const void* src, int64_t ld_src, int64_t src_rows, const int32_t* idx, void* dst,
                    int64_t ld_dst, int64_t rows, int64_t cols, void* stream);

/* ------------------------------------------------------------------ Wan2.2 VAE encoder (first frame)
 * Activations are channels-last rows (one row per pixel, [h*w, C] bf16); the convolutions are
 * fam_gemm calls over these rows (1x1) or over an im2col operand (3x3) whose row is the pixel's
 * neighbourhood with the taps outermost, (kh*3 + kw)*C + c, zero-padded to kpad columns.  The
 * reference's causal 3-D convolutions see only their last temporal tap on the first frame
 * (two zero frames in front, no cache): CausalConv3d FB/wan_video_vae.py:33-52.
 */

/*
 * fam_vae_patch_im2col -- conv1's operand straight from the image: img [3, H, W] bf16
 * (channel-first), patchified 2x2 to 12 channels c*4 + r*2 + q ('b c (h q) (w r) -> b (c r q) h w')
 * and gathered as the 3x3 neighbourhoods of the (H/2) x (W/2) grid: out [(H/2)*(W/2), 128],
 * columns (kh*3 + kw)*12 + channel, columns 108..127 zero.
 * Replaces: patchify FB/wan_video_vae.py:196-208 + Encoder3d_38.conv1's input :650, :680-695.
 */
int fam_vae_patch_im2col(const void* img, int64_t H, int64_t W, void* out, int64_t ldo, void* stream);

/*
 * fam_im2col3x3 -- out[p, (kh*3 + kw)*C + c] = x[y, x', c] around output pixel p of the H x W
 * channels-last grid x (row stride ldx); stride 1: 'same' zero padding (CausalConv3d's spatial
 * padding); stride 2: zero padding at the bottom / right only and (H/2) x (W/2) outputs
 * (ZeroPad2d((0, 1, 0, 1)) + Conv2d(3, stride 2) of Resample38 FB/wan_video_vae.py:245-262).
 * Columns 9*C..kpad-1 are zero.
 * Limits: C, ldx, kpad, ldo multiples of 8, kpad >= 9*C; 16-byte aligned; stride 2 needs even H, W.
 */
int fam_im2col3x3(const void* x, int64_t ldx, int64_t H, int64_t W, int64_t C, int64_t stride, void* out,
                  int64_t ldo, int64_t kpad, void* stream);

/*
 * fam_chan_rmsnorm -- y = act(x / max(||x||_2, 1e-12) * sqrt(C) * gamma) per row of C channels
 * (act FAM_ACT_NONE or FAM_ACT_SILU).
 * Replaces: RMS_norm FB/wan_video_vae.py:55-70 (channel_first, bias-free) and the nn.SiLU that
 *           follows it in ResidualBlock :274-278 and the encoder head :670-674.
 * Limits: C and strides multiples of 8; 16-byte aligned.
 */
int fam_chan_rmsnorm(const void* x, int64_t ldx, int64_t rows, int64_t C, const void* gamma, int act, void* y,
                     int64_t ldy, void* stream);

/*
 * fam_vae_avgdown -- AvgDown3D of one frame: x [H*W, Cin] channels-last; the frame axis is
 * front-padded with ft - 1 zero frames, ft x fs x fs blocks fold into channels c*F + t*fs*fs +
 * i*fs + j (F = ft*fs*fs) and output channel o is the mean of group [o*G, (o+1)*G), G =
 * Cin*F/Cout: out [(H/fs)*(W/fs), Cout], plus add [same layout, row stride ld_add] when non-null
 * (the sum with the last residual block's shortcut on a level without downsampling).
 * Replaces: AvgDown3D.forward FB/wan_video_vae.py:345-395 (the Down_ResidualBlock shortcut :442-474).
 * Limits: ft, fs in {1, 2}; fs divides H and W; Cout divides Cin*F.
 */
int fam_vae_avgdown(const void* x, int64_t ldx, int64_t H, int64_t W, int64_t Cin, int64_t Cout, int64_t ft,
                    int64_t fs, const void* add, int64_t ld_add, void* out, int64_t ldo, void* stream);

/*
 * fam_softmax_rows -- p = softmax(scale * s) per row, fp32 scores in, bf16 out.
 * Replaces: the softmax of the single-head F.scaled_dot_product_attention in AttentionBlock
 *           FB/wan_video_vae.py:321-342 (scores and P V are fam_gemm products around it).
 */
int fam_softmax_rows(const float* s, int64_t lds, int64_t rows, int64_t cols, float scale, void* p, int64_t ldp,
                     void* stream);

/*
 * fam_chan_affine_nchw -- out[c, p] = (x[p, c] - mean[c]) * inv_std[c]: the latent normalisation
 * of VideoVAE38_.encode with the channels-last rows written channel-first; mean and inv_std fp32.
 * Replaces: mu = (mu - scale[0]) * scale[1], FB/wan_video_vae.py:1313-1319.
 */
int fam_chan_affine_nchw(const void* x, int64_t ldx, int64_t P, int64_t C, const float* mean, const float* inv_std,
                         void* out, void* stream);

/*
 * fam_add_modulation -- out[t, l, :] = bf16(modulation[l, :] + t_mod[t, :]) for every
 * denoise step t < T and block l < L, vectors of length n (= 6 * hidden): the
 * `modulation + t_mod` of every block (FB/wan_video_dit.py:273-274, FB/mot.py:63-80).
 * Limits: n % 8 == 0.
 */
int fam_add_modulation(const void* t_mod, const void* modulation, void* out,
                       int64_t T, int64_t L, int64_t n, void* stream);

/*
 * fam_cae_decode -- the CAE-FastWAM action-VAE decoder, fp32 (CAm/action_ae.py:123-166, run in
 * fp32 by CA/fastwam.py:855-863): z [B, tokens, latent_dim] -> out [B, horizon, action_dim].
 *   x = in_w z + in_b (+ suite[b], the caller's suite embedding row, optional)
 *   for each of nstages strides s: ConvTranspose1d(C, C, 2s, stride s, padding s/2) ->
 *     GroupNorm(min(8, C)) -> SiLU -> x + GN(Conv1d_3(SiLU(GN(Conv1d_3(x)))))  (CAm/action_ae.py:32-48)
 *   time axis cropped / zero-padded to horizon, then out_w x + out_b per position.
 * Weights in PyTorch layouts: ConvTranspose1d [in, out, k], Conv1d [out, in, 3], Linear [out, in].
 * work: 3 * B * C * T floats of scratch (T = decoded length).  Limits: C <= 512 and divisible by
 * min(8, C); C * (T + 2) * 4 and (C T + action_dim C) * 4 bytes <= 64 KiB (T = decoded length), and per
 * stage (C T_in + 2 s C / G) * 4 <= 64 KiB; (C / G) * T <= 4096; nstages <= 3.
 */
typedef struct fam_cae_desc {
  const float* z; int64_t batch, tokens, latent_dim;
  const float* suite;
  int64_t hidden, horizon, action_dim, nstages; int64_t strides[3];
  const float* in_w; const float* in_b;
  const float* up_w[3]; const float* up_b[3]; const float* gn_w[3]; const float* gn_b[3];
  const float* r1_w[3]; const float* r1_b[3]; const float* rg1_w[3]; const float* rg1_b[3];
  const float* r2_w[3]; const float* r2_b[3]; const float* rg2_w[3]; const float* rg2_b[3];
  const float* out_w; const float* out_b;
  float* work; float* out;
  float gn_eps;
} fam_cae_desc;

int fam_cae_decode(const fam_cae_desc* d, void* stream);

/*
 * fam_tiny_expert -- the denoise loop of an action expert whose hidden width is 32 (the
 * CAE-FastWAM expert: hidden 32, 24 x 128 attention, 30 blocks; the compact expert of config 3:
 * hidden 32, 4 x 8 heads), in 2 launches per block step.  Phase p of the call (0 <= p <= 2 L T):
 *   p = 2 (t L + l)     self (MoT joint) attention sub-block of block l at step t,
 *   p = 2 (t L + l) + 1 cross-attention sub-block,
 *   p = 2 L T           the last block's FFN, the head and the last Euler update -> out.
 * The attention width A = heads * head_dim is cut into G = A / slice column slices of whole
 * heads; workgroup (g, b) of a phase owns slice g of batch row b:
 *   self:  completes the previous block (x += o_c + co_b, then x += gate_mlp FFN(AdaLN(x)))
 *          -- at l = 0 also the head, the Euler update of the chunk and the action encoder --
 *          then q, k, v of its heads from AdaLN(x), RMSNorm over all A columns (the sums of
 *          squares of the other slices from the layer's Gram matrix, gram below), 1-D RoPE,
 *          attention over [the layer's video K/V ; the action K/V] and its share of the o
 *          projection -> part_s[b, g];
 *   cross: x += gate_msa (sum_g part_s + o_b), then the slice's cross-attention query from the
 *          affine LayerNorm3 (RMSNorm as above), attention over the context and its share of
 *          the cross o projection -> part_c[b, g].  A 32-wide slice reads the context K/V
 *          (ctxkv, already RMS-normalised).  A wider slice attends in the 32-wide space of the
 *          context rows h (ctx_emb): with k = r (W_k h + b_k) * w_k (r the key's RMS factor over
 *          all A columns, w_k the key norm weight) the score of query q is
 *          r (h . W_k^T (q * w_k) + b_k . (q * w_k)), and the output
 *          sum p (W_v h + b_v) / l = W_v (sum p h / l) + b_v -- the same values with bf16
 *          rounding at other places; r comes from fam_tiny_context.
 * Every workgroup recomputes the [S, hidden] rows it needs from the previous phase's fp32
 * partials in a fixed order (no atomics, no communication within a launch); slice 0 stores
 * them for the next phase.  With G = 1 (A <= 128) the whole call is one launch per batch row.
 * Rounding: the residual stream and the chunk stay fp32; every product takes bf16 operands
 * with fp32 accumulation (as fam_gemm); q and k are rounded to bf16 after the norm and after
 * the rotation.
 *   gram (G > 1 or slice > 32): bf16 [L, 4, 2, 32, 32] -- hi and lo bf16 parts of W^T W for the
 *   self q, self k, cross q and cross k weights (W [A, 32] of the layer, as bf16 values); gram_c
 *   fp32 [L, 4, 32] = W^T b; gram_b fp32 [L, 4] = |b|^2.  Then sum_j q_j^2 = h G h + 2 c.h + |b|^2
 *   for the row h.
 *   video_k / video_v: device arrays of L pointers to [B, Sv, A] views with common strides.
 * Weights are layer-major stacks of the reference's nn.Linear layouts:
 *   qkv_w [L, 3A, 32] (q; k; v), qkv_b [L, 3A], nq_w / nk_w / cnq_w [L, A], o_w / co_w [L, 32, A],
 *   o_b / co_b / n3_w / n3_b / ff2_b [L, 32], cq_w [L, A, 32], cq_b [L, A], ff0_w [L, F, 32],
 *   ff0_b [L, F], ff2_w [L, 32, F]; enc_w [32, Da], enc_b [32], head_w [Da, 32], head_b [Da].
 *   mods bf16 [T, L, 6 * 32] = modulation + t_mod (shift, scale, gate of the attention; of the FFN).
 *   ctxkv bf16 [Lc, ctx_ld] (slice 32): block l's normalised keys at columns 2 A l, values at
 *   2 A l + A.  slice > 32 instead: ctx_emb bf16 [Lc, ctx_emb_ld] (the text embedding's rows),
 *   ck_wt [L, 32, A] (the cross key weight transposed), ck_b / cnk_w / cv_b [L, A], cv_w
 *   [L, A, 32], and ctx_rs fp32 [L, ceil(Lc / 32) * 32], which fam_tiny_context fills.
 *   rope_cos / rope_sin fp32 [S, head_dim / 2] (pair j of position s).
 * State (fp32, caller-owned): lat [2, B, S, Da], xa / xb [B, S, 32], part_s / part_c
 * [B, G, S, 32]; out [B, S, Da].  noise bf16 [B, S, Da] is read at phase 0.
 * fam_tiny_expert launches phases [phase_begin, phase_end) in order (one launch when G = 1).
 * Replaces: the action branch of MoT.forward per block step  FB/mot.py:378-478 (DiTBlock
 *           FB/wan_video_dit.py:267-286), its loop FB/fastwam.py:1051-1069, and the CAE tree's
 *           single-program ops for this expert: fastwam::mot_qkv_post, mot_attn_oproj,
 *           mot_ffn, mod_n3q, xattn_qn (CA/mot.py:2793-3010, 3227-3340, 3673-3760) with the
 *           time-independent parts of CA/action_dit.py:127-231.
 * Limits: hidden 32; S <= 16; slice in {32, 64, 128}, a multiple of head_dim, A % slice == 0,
 * (slice / head_dim) * S <= 32; head_dim a multiple of 8; F % 32 == 0, F <= 256; A / slice <= 64;
 * Da <= 32 and S * Da <= 256; 16-byte aligned weights, rows and strides (multiples of 8);
 * ctx_emb 8-byte aligned with ctx_emb_ld a multiple of 4.
 */
typedef struct fam_tiny_desc {
  int32_t batch, seq, hidden, heads, head_dim, ffn, action_dim, layers, steps, video_len, ctx_len, slice;
  float eps, scale;
  const void* noise; const void* mods; const void* deltas;
  const float* rope_cos; const float* rope_sin;
  const void* ctxkv; int64_t ctx_ld;
  const void* const* video_k; const void* const* video_v; int64_t video_bs, video_rs;
  const uint8_t* video_mask; int64_t mask_rs;
  const void* enc_w; const void* enc_b; const void* head_w; const void* head_b;
  const void* qkv_w; const void* qkv_b; const void* nq_w; const void* nk_w; const void* o_w; const void* o_b;
  const void* n3_w; const void* n3_b; const void* cq_w; const void* cq_b; const void* cnq_w;
  const void* co_w; const void* co_b; const void* ff0_w; const void* ff0_b; const void* ff2_w; const void* ff2_b;
  const void* gram; const float* gram_c; const float* gram_b;
  float* lat; float* xa; float* xb; float* part_s; float* part_c; float* out;
  const void* ctx_emb; int64_t ctx_emb_ld;
  const void* ck_wt; const void* ck_b; const void* cnk_w; const void* cv_w; const void* cv_b;
  float* ctx_rs;
  int32_t key_splits; float* part_x;
} fam_tiny_desc;

int fam_tiny_expert(const fam_tiny_desc* d, int64_t phase_begin, int64_t phase_end, void* stream);

/*
 * fam_tiny_key_splits -- the context splits KS that fam_tiny_expert's cross phases use for this
 * descriptor (a negative FAM_ERR_* when the descriptor is refused; part_x is not checked).
 * With one 32-wide slice (A = 32) and few batch rows a cross phase runs KS workgroups per batch
 * row, each over whole 32-key blocks of the context (key_splits = 0: the library's choice, at
 * most 8 splits of at least 4 blocks while B * KS fits the CUs; key_splits >= 1 asks for that
 * count, capped at 8 and at the context's blocks; either count then drops to the splits of
 * ceil(blocks / count) blocks that hold keys); each split stores its unnormalised output
 * with its running max and sum to part_x [B][KS][32][slice + 4] (fp32, caller-owned), and the
 * next phase merges the splits in split order before the cross o projection.
 * Replaces: no reference operation (the context attention of CrossAttention.forward,
 *           FB/wan_video_dit.py:214-219, split over workgroups).
 */
int fam_tiny_key_splits(const fam_tiny_desc* d);

/*
 * fam_tiny_context -- for slices wider than 32: every context key's factor
 * ctx_rs[l, i] = rsqrt(mean_j k_j^2 + eps) * scale * log2(e) of k = W_k h_i + b_k (block l's cross
 * key, all A columns, from the Gram form with gram[l, 3]); keys past Lc read row 0.  One launch;
 * run it whenever ctx_emb changes, before the first cross phase.  A 32-wide slice needs nothing
 * here (the call validates and returns FAM_OK).
 * Replaces: the per-call context keys' projection and RMSNorm k = norm_k(k(ctx))
 *           FB/wan_video_dit.py:216 (CrossAttention.forward) for every block.
 */
int fam_tiny_context(const fam_tiny_desc* d, void* stream);

/* Modes of fam_row_q8. */
#define FAM_Q8_ROW 0         /* y = x                                              */
#define FAM_Q8_GELU 1        /* y = bf16(GELU_tanh(x)), in the sigmoid form         */
#define FAM_Q8_LN_MOD 2      /* y = bf16(bf16(LN(x)) * (1 + scale) + shift)         */
#define FAM_Q8_ADD_LN_MOD 3  /* xo = bf16(x + x2); y = LN_MOD of xo                 */

/*
 * fam_row_q8 -- per-row fp8 quantisation of a row operation, one workgroup per row m < M:
 *   y as the mode says (LN: biased variance, fp32 statistics, (x - mean) / sqrt(var + eps));
 *   a = max |y| over the row;  s[m] = max(a, 1e-12) / 448;
 *   q[m, :] = fp8_e4m3(y * (448 / max(a, 1e-12)))   (OCP e4m3, round to nearest even).
 * x / x2 / xo bf16 [M, D] rows (16-byte aligned, strides multiples of 8), shift / scale bf16 [D]
 * broadcast over the rows, q 1-byte codes [M, D] (8-byte aligned rows), s fp32 [M].
 * Limits: 8 <= D <= 16384, D a multiple of 8.
 * Replaces: fastwam::row_q8, gelu_q8, ln_mod_q8, add_ln_mod_q8 (CA/mot.py:3763-3980), the
 *           activation side of the video prefill's fp8 GEMMs.
 */
typedef struct fam_rowq8_desc {
  int mode;
  const void* x; int64_t ldx;
  const void* x2; int64_t ldx2;
  const void* shift; const void* scale;
  float eps;
  void* y; int64_t ldy;
  float* s;
  void* xo; int64_t ldxo;
  int64_t M, D;
} fam_rowq8_desc;

int fam_row_q8(const fam_rowq8_desc* d, void* stream);

/*
 * fam_mask_bias -- additive attention-bias planes of the CAE action expert's masks:
 *   sb [MP, SKP] fp32: 0 where row m < M keeps key c (c < SK and am[m * SK + c] != 0), and for
 *      rows m >= M at key 0 only; -inf elsewhere;
 *   xb [MP, NCP] fp32 (skipped when NULL): 0 where m < M, c < NS and cm[m * cm_row_stride + c]
 *      != 0 (stride 0: one row for every m); -inf elsewhere.
 * am / cm are 1-byte masks (bool).  One launch for both planes.
 * Replaces: fastwam::mask_bias (CA/mot.py:3342-3369, kernel :2525-2560).
 */
int fam_mask_bias(const uint8_t* am, const uint8_t* cm, int64_t cm_row_stride, int64_t M, int64_t SK, int64_t NS,
                  int64_t MP, int64_t SKP, int64_t NCP, float* sb, float* xb, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FAM_HIP_H */
