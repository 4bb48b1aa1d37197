/*
 * trinix_attn.h -- C ABI of the MI355X (gfx950) attention-forward library
 * `libtrinix_attn.so`.
 *
 * Plain C: pointers, sizes and strides only, no torch or HIP types in the
 * signatures (streams travel as `void*`, a `hipStream_t`; NULL = the null
 * stream).  Every entry point is asynchronous on the given stream, allocates
 * no device memory, frees nothing, and returns a `trinix_status` code; no C++
 * exception crosses the boundary.  Tensors are owned by the caller.
 *
 * Strides are in ELEMENTS, in the reference's BSHD order
 * (batch, seq, head, head_dim) for q/k/v/out; the head_dim stride must be 1.
 * A head stride of 0 on k/v (an `expand`ed single KV head) is accepted.
 *
 * Reference interfaces replaced (paths relative to the trinix 0.1.4 tree):
 *   trinix_attn_fwd            <- TritonAttentionKernel.apply
 *                                 trinix/kernels/attention_kernel.py:497-664
 *                                 (launch of _fwd_kernel :234-434 and
 *                                 _fwd_kernel_with_mask :8-231)
 *   trinix_attn_fwd_splitkv,   <- TritonAttentionKernel.apply for seqlen_q != seqlen_k
 *   trinix_attn_fwd_splitkv_plan  (asserted away at attention_kernel.py:510; the
 *                                 layers' KV-cache decode, e.g.
 *                                 grouped_query_attention.py:179-187, runs the
 *                                 eager path base.py:347-400)
 *   trinix_attn_mask_blockmap  <- TritonAttentionKernel._prepare_mask
 *                                 trinix/kernels/attention_kernel.py:479-495
 *                                 (the (B,H,S,S) materialisation is replaced
 *                                 by a per-block classification of the mask)
 *   trinix_rope_apply          <- TritonRoPEKernel.apply / _apply_rope_pytorch
 *                                 trinix/kernels/rope_kernel.py:180-222,
 *                                 trinix/layers/embeddings/rope.py:111-134
 *   trinix_attn_bwd            <- no counterpart: the reference's Triton attention
 *                                 returns a detached output (attention_kernel.py:
 *                                 497-517); gradients of the eager path
 *                                 (trinix/layers/attention/base.py:347-400)
 *   trinix_qk_norm             <- q_norm / k_norm (FastRMSNorm over head_dim) after
 *                                 RoPE in the layers: base.py:163-176,
 *                                 grouped_query_attention.py:171-177,
 *                                 trinix/layers/norm/rmsnorm.py:62-75
 *   trinix_qk_layernorm        <- the same with qk_norm_type='layernorm' (FastLayerNorm
 *                                 over head_dim): base.py:167-169,
 *                                 trinix/layers/norm/layernorm.py:83-88
 *   trinix_qk_norm_bwd         <- the autograd backward of those eager modules and of
 *                                 the RoPE before them (rope.py:111-118), which the
 *                                 reference's layers train through
 *   trinix_alibi_bias          <- TritonALiBiKernel.apply / FastALiBiPositionEmbedding
 *                                 trinix/kernels/alibi_kernel.py:8-54,93-124,
 *                                 trinix/layers/embeddings/alibi.py:65-90
 *   trinix_attn_tile_config    <- calculate_attention_block_sizes
 *                                 trinix/kernels/utils.py:87-153
 *   trinix_attn_is_available   <- TritonAttentionKernel.is_available
 *                                 trinix/kernels/attention_kernel.py:470-477
 *   trinix_dropout_state_advance <- no counterpart: the generator state torch keeps for
 *                                 the eager path's F.dropout under graph capture
 *                                 (trinix/layers/attention/base.py:395)
 *   trinix_dropout_keep_map_bytes <- no counterpart: the size of the keep bits a dropout
 *                                 forward leaves for its backward, where the eager path
 *                                 keeps F.dropout's mask (base.py:395)
 */
#ifndef TRINIX_ATTN_H
#define TRINIX_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRINIX_ATTN_ABI_VERSION 6

typedef enum trinix_status {
  TRINIX_OK = 0,
  TRINIX_ERR_NULL_POINTER = 1,   /* a required pointer is NULL             */
  TRINIX_ERR_BAD_DTYPE = 2,      /* unsupported dtype / dtype mismatch      */
  TRINIX_ERR_BAD_HEAD_DIM = 3,   /* head_dim not built for the entry point (forward, backward: 64, 128, 256; split-KV: 64, 128) */
  TRINIX_ERR_BAD_SHAPE = 4,      /* non-positive or inconsistent sizes      */
  TRINIX_ERR_BAD_STRIDE = 5,     /* d-stride != 1, misaligned rows, or a 16-bit K/V key-row stride >= 2^22 elements */
  TRINIX_ERR_BAD_ARGUMENT = 6,   /* other invalid argument (dropout, ...)   */
  TRINIX_ERR_NO_DEVICE = 7,      /* no gfx950 device / HIP runtime error    */
  TRINIX_ERR_LAUNCH = 8,         /* hipGetLastError after the launch        */
  TRINIX_ERR_SCRATCH_TOO_SMALL = 9 /* the call needs more than the static scratch */
} trinix_status;

typedef enum trinix_dtype {
  TRINIX_F32 = 0,
  TRINIX_F16 = 1,
  TRINIX_BF16 = 2,
  TRINIX_U8 = 3 /* bool / uint8 masks only: value 0 or 1 is added */
} trinix_dtype;

/* Arguments of one attention forward.  Semantics (reference
 * trinix/kernels/attention_kernel.py:123-216):
 *   s[i,j] = scale * <q[b,i,hq], k[b,j,hkv]>
 *            - alibi[b,hq] * |i - j|          (if alibi_slopes)
 *            + mask[b,hq,i,j]                 (if mask)
 *   s[i,j] = -inf unless  j < seqlen_k,
 *                         j <= i              (if causal; top-left aligned),
 *                         -wl <= j - i <= wr  (if has_window)
 *   out[b,i,hq,:] = softmax_j(s[i,:]) @ v[b,:,hkv,:]
 *   hkv = hq / (nheads_q / nheads_kv)   (GQA/MQA without repeating KV)
 *   lse[b,hq,i] = log(sum_j exp(s[i,j]))  (natural log; optional)
 * Rows with no allowed key give NaN, as softmax over all -inf does.
 * bf16/fp16 calls without dropout sum the probabilities as rounded to the
 * input dtype for the P @ V product (the weights out is normalised by), so
 * their lse is within one unit roundoff of that dtype (2^-8 bf16, 2^-11
 * fp16) of the exact value; fp32, dropout and split-KV calls sum in fp32.
 */
typedef struct trinix_attn_fwd_args {
  const void* q;        /* (B, Sq, Hq, D)  */
  const void* k;        /* (B, Sk, Hkv, D) */
  const void* v;        /* (B, Sk, Hkv, D) */
  void* out;            /* (B, Sq, Hq, D), dtype of q */
  float* lse;           /* (B, Hq, Sq) fp32 contiguous, or NULL */
  int64_t q_stride[4];  /* b, s, h, d */
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t out_stride[4];
  int64_t batch, seqlen_q, seqlen_k, nheads_q, nheads_kv, head_dim;
  int32_t dtype;        /* trinix_dtype of q, k, v, out */
  float softmax_scale;
  int32_t causal;
  int32_t has_window;
  int64_t window_left, window_right;
  const float* alibi_slopes;    /* fp32, element (b, h) at b*s[0] + h*s[1]; NULL = none */
  int64_t alibi_stride[2];
  const void* mask;             /* additive mask, NULL = none */
  int32_t mask_dtype;           /* trinix_dtype */
  int64_t mask_stride[4];       /* b, h, i, j: each >= 0 (0 = broadcast), */
                                /* (seqlen_k-1)*j < 2^31, min(seqlen_q-1, 31)*i < 2^31 */
  const uint8_t* mask_blockmap; /* from trinix_attn_mask_blockmap, or NULL */
  int64_t blockmap_stride[2];   /* b, h strides of the block map (0 = broadcast) */
  /* Dropout on the attention weights: key j of row i of (b, h) is dropped
   * when 16-bit field j % 8 (word (j % 8) / 2, low half for even j) of
   * Philox4x32-10(counter (j / 8, i, b*H + h, offset_lo), key (seed_lo ^
   * offset_hi, seed_hi)) is below floor(p * 2^16); kept weights are scaled
   * by 1 / (1 - p). */
  float dropout_p;              /* 0 <= p < 1 */
  uint64_t dropout_seed;
  uint64_t dropout_offset;
  const void* rope_cos;         /* fused RoPE on q: cos/sin rows indexed by the  */
  const void* rope_sin;         /* query position, first D/2 columns used; dtype */
  int64_t rope_stride;          /* of q; NULL = no fused RoPE                    */
  /* Fused qk-norm of q (the layers' q RMSNorm over head_dim after RoPE,
   * reference trinix/layers/attention/grouped_query_attention.py:167-177):
   * each q row, after the fused RoPE if any, becomes
   * weight * dtype(h * rsqrt(mean(h^2) + eps)), with the rounding of
   * trinix_qk_norm, so q is bitwise the one trinix_qk_norm would write.
   * head_dim weights in q's dtype, 16-byte aligned; bf16/fp16 only, not
   * with a mask or dropout (TRINIX_ERR_BAD_ARGUMENT); NULL = none. */
  const void* q_norm_weight;
  float q_norm_eps;
  /* Dropout seed and offset in device memory (ABI version 5): two uint64,
   * {seed, offset}, 8-byte aligned, read by the kernels when they run in
   * place of dropout_seed / dropout_offset, so that a HIP graph replay can
   * draw new keep masks (trinix_dropout_state_advance writes them inside the
   * graph).  NULL = use dropout_seed / dropout_offset. */
  const uint64_t* dropout_state;
  /* With q_norm_weight (ABI version 5): the q the kernel attends with
   * (after the fused RoPE and RMSNorm) is also written here, a contiguous
   * (B, Sq, Hq, D) tensor of q's dtype, 16-byte aligned, so that a backward
   * (trinix_attn_bwd, then trinix_qk_norm_bwd) can use it.  NULL = not
   * written; requires q_norm_weight. */
  void* q_norm_out;
  /* Dropout keep map (ABI version 6): with dropout_p > 0 the forward also
   * writes its keep decisions here, one bit per (row, key), for a backward
   * to read instead of regenerating them (trinix_attn_bwd_args).  bf16/fp16
   * at head_dim 64 or 128 only (TRINIX_ERR_BAD_ARGUMENT otherwise), 16-byte
   * aligned, trinix_dropout_keep_map_bytes bytes.  Layout, per (b, h) in
   * order: 2*ceil(Sq/64) row blocks x 4*ceil(Sk/128) key blocks of 32 rows x
   * 32 keys; a block is 32 uint32 words, word i % 32 for row i, whose bit
   * 16h + 4q + e (h = 0, 1; q, e = 0..3) is set when key 8q + 4h + e of the
   * block is kept.  Words of rows, keys or key tiles the forward does not
   * visit (masked out, past Sq or Sk) are left as they were.
   * NULL = not written. */
  void* dropout_keep_map;
} trinix_attn_fwd_args;

/* Attention forward on `stream`. */
int trinix_attn_fwd(const trinix_attn_fwd_args* args, void* stream);

/* Split-KV forward for decode-shaped calls (seqlen_q <= 16 against a long
 * KV cache), same semantics and arguments as trinix_attn_fwd.  Extension:
 * the reference asserts seqlen_q == seqlen_k (attention_kernel.py:510) and
 * its layers' cache path runs the eager attention (base.py:347-400).
 * The rows of one KV head's q-heads are packed into 16-row tiles, and the
 * keys any row may see are cut into `num_splits` chunks merged by their
 * log-sum-exp.
 *
 * trinix_attn_fwd_splitkv_plan: *num_splits = 0 if the split-KV kernel does
 * not apply (fp32, dropout, fused RoPE or q norm, seqlen_q > 16, no visible
 * key): use
 * trinix_attn_fwd.  Otherwise the chunk count and the size of the fp32
 * workspace trinix_attn_fwd_splitkv needs (0 for a single chunk).  Host
 * only, no launch.
 * trinix_attn_fwd_splitkv: the forward on `stream`; `workspace` is
 * caller-owned device memory of at least the planned size, 16-byte aligned
 * (may be NULL when the plan asks for 0 bytes).  Returns
 * TRINIX_ERR_BAD_ARGUMENT where the plan does not apply or the workspace is
 * too small. */
int trinix_attn_fwd_splitkv_plan(const trinix_attn_fwd_args* args,
                                 int32_t* num_splits,
                                 int64_t* workspace_bytes);
int trinix_attn_fwd_splitkv(const trinix_attn_fwd_args* args, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* trinix_attn_fwd_splitkv without a workspace argument and without any
 * allocation: no counterpart in the reference.  It is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The partial results go to a
 * static device array of TRINIX_SPLITKV_SCRATCH_BYTES that the library holds
 * on every GPU it runs on until the process ends (its address is looked up
 * once per device).  Same arguments, semantics and output as
 * trinix_attn_fwd_splitkv; `stream` must belong to the current device
 * (TRINIX_ERR_BAD_ARGUMENT otherwise, before any launch).
 * Returns TRINIX_ERR_SCRATCH_TOO_SMALL when the plan's workspace exceeds the
 * array (the default plan needs at most about 17 MB), before any launch.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (different streams, or host threads) race and must be serialised by
 * the caller.  Every partial a call reads is written by the same call, so
 * nothing needs clearing between calls. */
#define TRINIX_SPLITKV_SCRATCH_BYTES (32u << 20)
int trinix_attn_fwd_splitkv_noalloc(const trinix_attn_fwd_args* args, void* stream);

/* Block classification of an additive mask of logical size
 * (mb, mh, seqlen_q, seqlen_k) with element strides `stride` (0 = broadcast).
 * Writes out[((b*mh + h)*ceil(Sq/32) + r)*ceil(Sk/64) + c] for each 32x64
 * block: 0 = every element is +0/-0 (no load needed), 2 = every element is
 * -inf (block skipped), 1 = anything else (loaded per element). */
int trinix_attn_mask_blockmap(const void* mask, int32_t mask_dtype,
                              int64_t mb, int64_t mh, int64_t seqlen_q,
                              int64_t seqlen_k, const int64_t stride[4],
                              uint8_t* out, void* stream);
/* Rows and columns covered by one block-map entry. */
#define TRINIX_BLOCKMAP_ROWS 32
#define TRINIX_BLOCKMAP_COLS 64

/* Rotary embedding, reference trinix/layers/embeddings/rope.py:111-134:
 *   out = x*cos + rotate_half(x)*sin, rotate_half(x) = cat(-x2, x1),
 * with every product and the sum rounded to the tensor dtype, as eager
 * PyTorch does.  x, out: (B, S, H, D) with strides (d stride 1); cos/sin:
 * rows of >= D/2 entries in x's dtype with row stride `cs_stride`; row
 * index = position_ids[b*S + s] (int64) if position_ids != NULL, else s.
 * `cs_rows` is the number of table rows (>= seqlen without position_ids);
 * position ids outside [0, cs_rows) are clamped into it, so no id reads
 * outside the tables (host wrappers reject such ids where they can read
 * them, i.e. outside graph capture). */
int trinix_rope_apply(const void* x, const int64_t x_stride[4], void* out,
                      const int64_t out_stride[4], int64_t batch,
                      int64_t seqlen, int64_t nheads, int64_t head_dim,
                      int32_t dtype, const void* cos, const void* sin,
                      int64_t cs_stride, int64_t cs_rows,
                      const int64_t* position_ids, void* stream);

/* qk-norm of the attention layers, fused with RoPE (reference
 * trinix/layers/attention/base.py:163-176 with FastRMSNorm's PyTorch path
 * trinix/layers/norm/rmsnorm.py:62-75, applied after RoPE at
 * grouped_query_attention.py:171-177):
 *   y   = cos ? rope(x) : x          (as trinix_rope_apply, rounded to dtype)
 *   out = weight * to_dtype(y * rsqrt(mean_d(y^2) + eps))
 * bf16/fp16 x, out and weight (head_dim elements, same dtype); head_dim in
 * {16, 32, 64, 128, 256}; x/out (B, S, H, D) element strides, d stride 1,
 * 16-byte aligned rows; cos/sin/cs_rows/position_ids as for
 * trinix_rope_apply.  The fp32 sum of
 * squares is ordered differently from torch's reduction: an output element
 * can differ from eager by one ulp of the dtype, rarely. */
int trinix_qk_norm(const void* x, const int64_t x_stride[4], void* out,
                   const int64_t out_stride[4], int64_t batch, int64_t seqlen,
                   int64_t nheads, int64_t head_dim, int32_t dtype,
                   const void* weight, float eps, const void* cos,
                   const void* sin, int64_t cs_stride, int64_t cs_rows,
                   const int64_t* position_ids, void* stream);

/* LayerNorm variant of trinix_qk_norm (reference qk_norm_type='layernorm',
 * trinix/layers/attention/base.py:167-169: FastLayerNorm's PyTorch path
 * trinix/layers/norm/layernorm.py:83-88, F.layer_norm with weight and bias
 * cast to the input dtype):
 *   y   = cos ? rope(x) : x
 *   out = to_dtype((y - mean_d(y)) * rsqrt(var_d(y) + eps) * weight + bias)
 * in fp32 (biased variance); weight and bias of head_dim elements in the
 * dtype of x.  Other arguments as for trinix_qk_norm.  ABI version 4. */
int trinix_qk_layernorm(const void* x, const int64_t x_stride[4], void* out,
                        const int64_t out_stride[4], int64_t batch,
                        int64_t seqlen, int64_t nheads, int64_t head_dim,
                        int32_t dtype, const void* weight, const void* bias,
                        float eps, const void* cos, const void* sin,
                        int64_t cs_stride, int64_t cs_rows,
                        const int64_t* position_ids, void* stream);

/* norm_type of trinix_qk_norm_bwd */
#define TRINIX_NORM_RMS 0   /* trinix_qk_norm */
#define TRINIX_NORM_LAYER 1 /* trinix_qk_layernorm */

/* Backward of trinix_qk_norm / trinix_qk_layernorm: the gradients eager
 * autograd gives through the RoPE and the norm modules the reference's
 * layers train with (base.py:163-176, rmsnorm.py:62-75, layernorm.py:83-88,
 * rope.py:111-118).  x is the forward's input (before RoPE), dout the
 * gradient of its output; dx (same layout rules as x) receives the gradient
 * of x.  dweight_partial (and, for TRINIX_NORM_LAYER, dbias_partial) are
 * caller-provided fp32 arrays of partial_rows x head_dim elements: row r
 * receives the column sums of workgroup r (partial_rows workgroups walk the
 * rows; any partial_rows >= 1 is valid).  The caller adds the rows and
 * rounds to the weight's dtype to get dweight (dbias).  eps, weight, cos,
 * sin, cs_stride, cs_rows and position_ids are the forward's.  ABI
 * version 4. */
int trinix_qk_norm_bwd(const void* x, const int64_t x_stride[4],
                       const void* dout, const int64_t dout_stride[4],
                       void* dx, const int64_t dx_stride[4], int64_t batch,
                       int64_t seqlen, int64_t nheads, int64_t head_dim,
                       int32_t dtype, int32_t norm_type, const void* weight,
                       float eps, const void* cos, const void* sin,
                       int64_t cs_stride, int64_t cs_rows,
                       const int64_t* position_ids, float* dweight_partial,
                       float* dbias_partial, int64_t partial_rows,
                       void* stream);

/* Backward of trinix_attn_fwd.  No counterpart in the reference (its
 * Triton attention has no backward, attention_kernel.py:497-517); the
 * gradients are those of the eager path
 * dropout(softmax(scale*q k^T + ALiBi + mask)) v (base.py:347-400):
 *   P  = softmax(z),  Pd = P * keep / (1 - dropout_p)
 *   dv = Pd^T dout,  dz = P*(keep*(dout v^T)/(1 - dropout_p) - rowsum(dout*out)),
 *   dq = scale*dz k,  dk = scale*dz^T q (summed over the q-heads sharing a KV head).
 * keep is the forward's dropout mask, regenerated from the same
 * dropout_seed / dropout_offset (pass those of the forward call).
 * dtype fp32, bf16 or fp16; head_dim 64, 128 or 256.
 * q, k, v, out, dout and the outputs dq (like q), dk, dv (like k, v) are
 * BSHD with d stride 1; lse is the (B, Hq, Sq) fp32 natural-log row
 * log-sum-exp written by trinix_attn_fwd; delta is a caller-provided fp32
 * workspace of B*Hq*Sq elements.  Scale, causal, window, ALiBi and mask
 * arguments mean what they mean in trinix_attn_fwd_args.  ABI version 3
 * appended the three dropout fields. */
typedef struct trinix_attn_bwd_args {
  const void* q;
  const void* k;
  const void* v;
  const void* out;
  const void* dout;
  const float* lse;
  float* delta;
  void* dq;
  void* dk;
  void* dv;
  int64_t q_stride[4];
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t out_stride[4];
  int64_t dout_stride[4];
  int64_t dq_stride[4];
  int64_t dk_stride[4];
  int64_t dv_stride[4];
  int64_t batch, seqlen_q, seqlen_k, nheads_q, nheads_kv, head_dim;
  int32_t dtype;
  float softmax_scale;
  int32_t causal;
  int32_t has_window;
  int64_t window_left, window_right;
  const float* alibi_slopes;
  int64_t alibi_stride[2];
  const void* mask;
  int32_t mask_dtype;
  int64_t mask_stride[4];      /* as in trinix_attn_fwd_args */
  const uint8_t* mask_blockmap;
  int64_t blockmap_stride[2];
  float dropout_p;              /* the forward's dropout_p, seed and offset */
  uint64_t dropout_seed;
  uint64_t dropout_offset;
  const uint64_t* dropout_state; /* the forward's, as in trinix_attn_fwd_args */
  /* The keep map the forward wrote (ABI version 6), read in place of
   * regenerating the keep mask: bf16/fp16 at head_dim 64 or 128 with
   * dropout_p > 0 only (TRINIX_ERR_BAD_ARGUMENT otherwise).  NULL =
   * regenerate from dropout_seed / dropout_offset / dropout_state. */
  const void* dropout_keep_map;
} trinix_attn_bwd_args;
int trinix_attn_bwd(const trinix_attn_bwd_args* args, void* stream);

/* ALiBi bias, reference trinix/kernels/alibi_kernel.py:8-54:
 *   out[h*out_stride_h + i*out_stride_i + j] = -slopes[h*slope_stride] * |i - j|
 * for h < nheads, i, j < seqlen (< 2^24), fp32, key stride 1. */
int trinix_alibi_bias(const float* slopes, int64_t slope_stride, int64_t nheads,
                      int64_t seqlen, float* out, int64_t out_stride_h,
                      int64_t out_stride_i, void* stream);

/* Tile shape the library launches for (head_dim, dtype). */
typedef struct trinix_tile_cfg {
  int32_t block_m;      /* query rows per workgroup (large-problem shape) */
  int32_t block_n;      /* keys per K/V tile            */
  int32_t block_d;      /* head_dim the kernel runs at  */
  int32_t waves;        /* wavefronts per workgroup     */
  int32_t lds_bytes;    /* LDS per workgroup            */
} trinix_tile_cfg;
int trinix_attn_tile_config(int64_t head_dim, int32_t dtype, trinix_tile_cfg* out);

/* 1 if a gfx950 device is visible to the HIP runtime, else 0. */
int trinix_attn_is_available(void);

/* Static description of a status code. */
const char* trinix_status_string(int status);

/* Dropout under HIP graph capture: no counterpart in the reference, whose
 * eager dropout (trinix/layers/attention/base.py:395, F.dropout) takes its
 * seed and offset from torch's graph-safe generator state.  Copies
 * generator[0..1] = {seed, offset} to call_state[0..1] and advances
 * generator[1] by `increment`, in one single-lane kernel on `stream`: a
 * call captured in a graph then draws a new offset on every replay, and the
 * forward and backward of that call read the same call_state.  Both
 * pointers are device memory, 8-byte aligned, two uint64 each. */
int trinix_dropout_state_advance(uint64_t* generator, uint64_t* call_state, uint64_t increment, void* stream);

/* Size in bytes of the dropout keep map of a (batch, nheads_q, seqlen_q,
 * seqlen_k) attention: 128 * batch * nheads_q * 2*ceil(seqlen_q/64) *
 * 4*ceil(seqlen_k/128).  No counterpart in the reference, whose eager path
 * keeps F.dropout's mask of the attention weights for its backward
 * (trinix/layers/attention/base.py:395) at one element per (row, key). */
int trinix_dropout_keep_map_bytes(int64_t batch, int64_t nheads_q, int64_t seqlen_q, int64_t seqlen_k,
                                  int64_t* bytes);

/* TRINIX_ATTN_ABI_VERSION of the built library. */
int trinix_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* TRINIX_ATTN_H */
