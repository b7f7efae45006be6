/*
 * prefixlm.h -- C ABI of the MI355X (gfx950) packed varlen PrefixLM attention.
 *
 * This library replaces the FlashAttention-3 calls behind HRM-Text's
 * `flash_attn_varlen_prefixlm` (reference: models/flash_attention_prefixlm_v2.py).
 * It exposes plain pointers, strides and sizes only; it never allocates device
 * memory: outputs and a scratch workspace are passed in by the caller.
 *
 * Shapes: T = rows of q (the padded packed token count), H = heads, D = head dim.
 *   q, k, v, out, dout, dq, dk, dv : bf16 [T, H, D], unit stride over D,
 *                                    element strides over tokens (_stride_t) and heads (_stride_h)
 *   lse                            : float32 [H, T], natural log of the sum of exp(scale * q.k)
 *                                    over the keys a row attends; -inf on rows >= total_seqlen
 *   prefix_lens, causal_lens, cu_seqlens : int32 device arrays in the reference's padded format
 *                                    (models/flash_attention_prefixlm_v2.py:10-24), length meta_len
 *
 * Masking: query i of a segment with prefix p attends key j of the same segment iff
 * j <= i or j < p (j <= i when is_causal). Rows >= total_seqlen get zero outputs/grads.
 *
 * Every entry point returns 0 on success and a nonzero prefixlm_status otherwise;
 * prefixlm_last_error() then describes the failure (thread-local string).
 * Launches are asynchronous on `stream` (a hipStream_t; NULL = default stream).
 */
#ifndef PREFIXLM_H_
#define PREFIXLM_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum prefixlm_status {
  PREFIXLM_OK = 0,
  PREFIXLM_ERR_INVALID = 1,   /* bad shape, stride, alignment, size or workspace */
  PREFIXLM_ERR_HIP = 2,       /* a HIP runtime call or kernel launch failed */
  PREFIXLM_ERR_METADATA = 3   /* prefixlm_check_workspace: kernels saw inconsistent metadata */
} prefixlm_status;

typedef struct prefixlm_fwd_args {
  uint32_t struct_size;          /* sizeof(prefixlm_fwd_args) as the caller compiled it: calls
                                    with another value (a caller built against another version
                                    of this header) are rejected */
  const void* q;                 /* bf16 */
  const void* k;
  const void* v;
  void* out;                     /* bf16 [T, H, D] */
  void* out_lo;                  /* optional (NULL = skip): int8 [T, H, D] rounding residual of
                                    the fp32 result O, for a precise backward: with out = m 2^e
                                    (m in [0.5, 1)), out_lo = clamp(rint((O - out) 2^(16-e)),
                                    -128, 127), so out + out_lo 2^(e-16) is O to ~16 bits.
                                    Strides (in elements = bytes) multiples of 16 */
  float* lse;                    /* float32 [H, T], contiguous */
  int64_t q_stride_t, q_stride_h;
  int64_t k_stride_t, k_stride_h;
  int64_t v_stride_t, v_stride_h;
  int64_t out_stride_t, out_stride_h;
  int64_t out_lo_stride_t, out_lo_stride_h;
  const int32_t* prefix_lens;    /* device */
  const int32_t* causal_lens;    /* device */
  const int32_t* cu_seqlens;     /* device */
  int64_t meta_len;              /* length of the three metadata arrays */
  int32_t num_tokens;            /* T */
  int32_t num_heads;             /* H */
  int32_t head_dim;              /* D: 128, or 64 (kernels of its own; no gate) */
  int32_t total_seqlen;          /* host scalars of the reference op (:103-108) */
  int32_t numseqs;
  int32_t max_seqlen_prefix;
  int32_t max_seqlen_causal;
  int32_t max_seqlen_all;
  int32_t is_causal;             /* nonzero: plain causal within each segment */
  float softmax_scale;           /* e.g. 1/sqrt(D) */
  void* workspace;               /* device scratch, >= prefixlm_fwd_workspace_size(...) bytes
                                    (the work list); unused (may be NULL) when `plan` is given */
  size_t workspace_bytes;
  const void* plan;              /* optional (NULL = build the work list on the device): a plan from
                                    prefixlm_plan_build for this batch, copied to the device */
  size_t plan_bytes;
  const void* gate;              /* optional (NULL = none): bf16 [T, H, D] output gate of the attention
                                    layer (models/layers.py:154); then also */
  void* out_gated;               /* bf16 [T, H, D] = sigmoid(gate) * out, 0 on rows >= total_seqlen */
  int64_t gate_stride_t, gate_stride_h;
  int64_t out_gated_stride_t, out_gated_stride_h;
  void* timer;                   /* optional (NULL = none): a prefixlm_timer_create() handle that
                                    records HIP events around each launch of this call */
  float* q_amax;                 /* optional (NULL = skip; the backward needs it): float32,
                                    prefixlm_fwd_q_amax_count(num_tokens, num_heads) slots, of
                                    which the call writes max |q| over the rows of each wave of
                                    its grid (0 for none), for the backward's fp16 scale of q.
                                    Requires numseqs <= num_tokens */
} prefixlm_fwd_args;

typedef struct prefixlm_bwd_args {
  uint32_t struct_size;          /* sizeof(prefixlm_bwd_args), checked as in prefixlm_fwd_args */
  const void* q;
  const void* k;
  const void* v;
  const void* out;               /* forward output */
  const void* out_lo;            /* optional (NULL = none): forward's out_lo (int8) */
  const void* dout;              /* gradient of out */
  const float* lse;              /* forward LSE [H, T] */
  const float* q_amax;           /* the forward's q_amax (required) */
  void* dq;                      /* bf16 [T, H, D] */
  void* dk;
  void* dv;
  int64_t q_stride_t, q_stride_h;
  int64_t k_stride_t, k_stride_h;
  int64_t v_stride_t, v_stride_h;
  int64_t out_stride_t, out_stride_h;
  int64_t out_lo_stride_t, out_lo_stride_h;
  int64_t dout_stride_t, dout_stride_h;
  int64_t dq_stride_t, dq_stride_h;
  int64_t dk_stride_t, dk_stride_h;
  int64_t dv_stride_t, dv_stride_h;
  const int32_t* prefix_lens;
  const int32_t* causal_lens;
  const int32_t* cu_seqlens;
  int64_t meta_len;
  int32_t num_tokens;
  int32_t num_heads;
  int32_t head_dim;
  int32_t total_seqlen;
  int32_t numseqs;
  int32_t max_seqlen_prefix;
  int32_t max_seqlen_causal;
  int32_t max_seqlen_all;
  int32_t is_causal;
  float softmax_scale;
  void* workspace;               /* >= prefixlm_bwd_workspace_size(...) bytes */
  size_t workspace_bytes;
  const void* plan;              /* optional, as in prefixlm_fwd_args */
  size_t plan_bytes;
  const void* gate;              /* optional (NULL = none): the forward's gate. Then `dout` is the
                                    gradient of out_gated, and the call also writes */
  void* dgate;                   /* bf16 [T, H, D], the gradient of gate (0 on rows >= total_seqlen) */
  void* dout_attn;               /* bf16 [T, H, D] scratch: dout * sigmoid(gate), the gradient of out */
  int64_t gate_stride_t, gate_stride_h;
  int64_t dgate_stride_t, dgate_stride_h;
  int64_t dout_attn_stride_t, dout_attn_stride_h;
  void* timer;                   /* optional, as in prefixlm_fwd_args */
  void* ds_buf;                  /* optional (NULL = none): 256-byte aligned, >= prefixlm_bwd_ds_bytes(...)
                                    bytes, or >= prefixlm_bwd_ds_bytes_blocks(..., ds_blocks) with
                                    ds_blocks set. With it the dK/dV kernel also stores dS and dQ is
                                    computed from the stored dS instead of recomputing S, P and dP;
                                    without it (or when the size function gives 0) the recomputing
                                    dQ kernel runs. */
  size_t ds_buf_bytes;
  int64_t ds_blocks;             /* stored-dS blocks per head the buffer holds: 0 = the bound
                                    prefixlm_bwd_ds_bytes derives from max_seqlen_all; with a plan,
                                    prefixlm_plan_ds_blocks(plan) sizes it to exactly the blocks
                                    the call writes. A batch that needs more is flagged in the
                                    workspace's error word (device-built lists). */
} prefixlm_bwd_args;

/* Slots (floats) of prefixlm_fwd_args.q_amax: one per wave of the forward's grid for any
 * batch of num_tokens rows (66 k floats per head for 16384 tokens). No counterpart
 * in the reference: the backward computes the dK product in fp16 with q scaled by a
 * power of two from these maxima (bf16 to fp16 is then exact). */
size_t prefixlm_fwd_q_amax_count(int32_t num_tokens, int32_t num_heads);

/* Workspace bytes for one forward / backward call with these host scalars. */
size_t prefixlm_fwd_workspace_size(int32_t num_tokens, int32_t num_heads, int32_t head_dim,
                                   int32_t total_seqlen, int32_t numseqs);
size_t prefixlm_bwd_workspace_size(int32_t num_tokens, int32_t num_heads, int32_t head_dim,
                                   int32_t total_seqlen, int32_t numseqs);
/* Bytes of the optional dS buffer of prefixlm_bwd. The buffer holds, per head, one fp16
 * block of 32 queries x 64 keys for every attended (32-row query tile, 64-key group) pair
 * of every segment (2 bytes per attended (query, key) pair, rounded up to whole blocks),
 * plus one scale per 128-key tile. The host scalars alone only bound the block count:
 * prefixlm_bwd_ds_bytes sizes for every 32-row tile times ceil(max_seqlen_all / 64) key
 * groups (about 2 * num_heads * num_tokens * max_seqlen_all bytes), while
 * prefixlm_bwd_ds_bytes_blocks sizes for a given block count per head, e.g. the exact one
 * of a plan (prefixlm_plan_ds_blocks; 0.54 GB for 16384 tokens, 16 heads and the
 * log-normal segments of the benchmark). Both give 0 when one head's blocks would not fit
 * 32-bit offsets (2 GiB) or a segment is longer than 32768: the call then ignores ds_buf.
 * No counterpart in the reference (FA3 recomputes in its dQ pass). */
size_t prefixlm_bwd_ds_bytes(int32_t num_tokens, int32_t num_heads, int32_t numseqs, int32_t max_seqlen_all);
size_t prefixlm_bwd_ds_bytes_blocks(int32_t num_tokens, int32_t num_heads, int32_t numseqs, int64_t ds_blocks);

/* Forward: out and lse for all T rows (both FA3 passes and the padding fill of
 * flash_attn_varlen_prefixlm_compileop, models/flash_attention_prefixlm_v2.py:88-131).
 * The reference returns two half-valid LSE tensors (:131); this returns one merged LSE. */
int prefixlm_fwd(const prefixlm_fwd_args* args, void* stream);

/* Backward: dq, dk, dv for all T rows (flash_attn_varlen_prefixlm_bwd_compileop,
 * models/flash_attention_prefixlm_v2.py:152-212, including dk1+dk2 / dv1+dv2 and the
 * zeroed padding rows). Uses the merged LSE of prefixlm_fwd. */
int prefixlm_bwd(const prefixlm_bwd_args* args, void* stream);

/* Backward that allocates nothing and takes no workspace: the same kernels as prefixlm_bwd,
 * with their scratch (work lists, statistics, delta) in a fixed array the library holds on
 * each GPU (prefixlm_bwd_noalloc_max_scratch() bytes, 16 MiB, kept until the process ends).
 * No counterpart in the reference: for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc). Capturing it in a HIP graph has not
 * been verified.
 * `workspace` must be NULL and workspace_bytes 0, `timer` NULL. Calls whose
 * prefixlm_bwd_workspace_size(...) exceeds the scratch are rejected (PREFIXLM_ERR_INVALID;
 * e.g. num_heads * num_tokens above ~4M at head_dim 128). Every call on one GPU shares
 * that GPU's scratch: calls that overlap on one GPU (other streams or threads) race. The
 * kernels rewrite everything they read from it, so nothing carries over between calls. */
size_t prefixlm_bwd_noalloc_max_scratch(void);
int prefixlm_bwd_noalloc(const prefixlm_bwd_args* args, void* stream);

/* Work-list plan: the cost-ordered tile lists that prefixlm_fwd / prefixlm_bwd otherwise
 * build on the device at every call, computed on the host from host copies of the batch
 * metadata (no GPU call; e.g. in the data loader next to compute_aux_seq_tensors_scalars,
 * dataset_new.py:129-134). Copy it to the device (256-byte aligned) and pass it in the
 * args of every call on that batch: the calls then skip the work-list kernel. The plan is
 * valid for either value of is_causal (is_causal only orders the lists). A plan whose
 * size does not fit the call's total_seqlen/numseqs is rejected; one built from other
 * metadata of the same size gives wrong results (items naming segments >= numseqs are
 * skipped, so nothing is read out of bounds). No counterpart in the reference, which
 * sizes its FA3 grids from the max_seqlen scalars instead
 * (models/flash_attention_prefixlm_v2.py:115-128). */
size_t prefixlm_plan_size(int32_t total_seqlen, int32_t numseqs);
/* prefix_lens / causal_lens / cu_seqlens: host arrays (>= numseqs, numseqs, numseqs+1
 * entries) in the reference's format. Returns PREFIXLM_ERR_METADATA for inconsistent
 * segments (the checks prefixlm_check_workspace reports for device-built lists). */
int prefixlm_plan_build(const int32_t* prefix_lens, const int32_t* causal_lens, const int32_t* cu_seqlens,
                        int32_t numseqs, int32_t total_seqlen, int32_t num_tokens, int32_t is_causal,
                        void* plan, size_t plan_bytes);
/* Stored-dS blocks per head of the batch a host plan was built for (the ds_blocks to pass
 * with it), or -1 if `plan` is not a plan of plan_bytes bytes. */
int64_t prefixlm_plan_ds_blocks(const void* plan, size_t plan_bytes);

/* Rotary position embedding of the reference's attention layer (apply_rotary_pos_emb,
 * models/layers.py:23-38, applied to q and k at :138-140), half-split layout, fp32
 * arithmetic in the reference's operation order (bitwise its result), or its transpose
 * for the backward. x, y: bf16 [T, heads, 128] (y may be x); cos, sin: fp32 [T, 128]
 * rows, the gathered cos_sin of RotaryEmbedding (:41-60). */
typedef struct prefixlm_rope_args {
  const void* x;
  void* y;
  const float* cos;
  const float* sin;
  int64_t x_stride_t, x_stride_h;
  int64_t y_stride_t, y_stride_h;
  int64_t cs_stride_t;           /* element stride between cos (and sin) rows */
  int32_t num_tokens;
  int32_t num_heads;
  int32_t head_dim;              /* 128 */
  int32_t backward;              /* 0: y = rope(x); nonzero: y = rope^T(x), the gradient map */
} prefixlm_rope_args;
int prefixlm_rope(const prefixlm_rope_args* args, void* stream);

/* SwiGLU activation of the block's MLP (models/layers.py:166-168, `F.silu(gate) * up` on
 * the two halves of the gate/up projection). gu: bf16 [rows, 2*cols], gate = columns
 * [0, cols), up = columns [cols, 2*cols). Forward: y [rows, cols] = silu(gate) * up.
 * Backward: dgu [rows, 2*cols] = [dy * up * s * (1 + gate * (1 - s)), dy * silu(gate)] with
 * s = sigmoid(gate), the gradient of the whole projection output (no concatenation needed).
 * fp32 arithmetic, one bf16 rounding per output. Unit column stride; row strides in
 * elements, multiples of 8; cols % 8 == 0; pointers 16-byte aligned. */
typedef struct prefixlm_swiglu_args {
  const void* gu;
  const void* dy;                /* backward only: bf16 [rows, cols] */
  void* y;                       /* forward output: bf16 [rows, cols] */
  void* dgu;                     /* backward output: bf16 [rows, 2*cols] */
  int64_t gu_stride, y_stride, dy_stride, dgu_stride;
  int64_t rows;
  int64_t cols;
} prefixlm_swiglu_args;
int prefixlm_swiglu_fwd(const prefixlm_swiglu_args* args, void* stream);
int prefixlm_swiglu_bwd(const prefixlm_swiglu_args* args, void* stream);

/* Weightless RMSNorm of the pre-norm block (models/transformer.py:87, `F.rms_norm(x, (N,),
 * eps)` over the last dimension). Forward: y = x * rstd with rstd = (mean(x^2) + eps)^-1/2 per
 * row, stored in fp32 [rows] for the backward. Backward: dx = rstd * dy - x * rstd^3 *
 * mean(dy * x). bf16 x, y, dy, dx with unit column stride and row strides that are multiples
 * of 8; 8 <= cols <= 8192, cols % 8 == 0. y may be x and dx may be dy. */
typedef struct prefixlm_rmsnorm_args {
  const void* x;
  const void* dy;                /* backward only */
  void* y;                       /* forward output */
  void* dx;                      /* backward output */
  float* rstd;                   /* fp32 [rows]: written by the forward, read by the backward */
  int64_t x_stride, y_stride, dy_stride, dx_stride;
  int64_t rows;
  int32_t cols;
  float eps;
} prefixlm_rmsnorm_args;
int prefixlm_rmsnorm_fwd(const prefixlm_rmsnorm_args* args, void* stream);
int prefixlm_rmsnorm_bwd(const prefixlm_rmsnorm_args* args, void* stream);

/* Projection GEMM of the block with the pre-norm RMSNorm fused in, and optionally the MLP's
 * SwiGLU (models/transformer.py:87-92, models/layers.py:124-135, :158-168):
 *   swiglu = 0: y = rmsnorm(x) W^T                         (y: [M, N])
 *   swiglu = 1: y = silu(rmsnorm(x) Wg^T) * (rmsnorm(x) Wu^T)  (W = [Wg; Wu], N = 2F, y: [M, F])
 * rmsnorm is the weightless F.rms_norm(x, (K,), eps) when norm != 0, the identity
 * otherwise; it is applied as the per-row scale it is: a row pass writes the scales
 * r = (mean(x^2) + eps)^(-1/2) to `rstd` (M floats, required with norm; F.rms_norm's
 * rstd, which its backward reuses) and the GEMM multiplies its fp32 products by them,
 * so the normalized x and the [M, 2F] gate/up product are never written. Forward only
 * (the reference computes these under torch.no_grad for all but the last bp_steps module
 * calls). bf16 x [M, K], W [N, K], y; unit column strides; row strides in elements,
 * multiples of 8; K % 64 == 0 (and K <= 8192 with norm); N % 256 == 0; fp32
 * accumulation, one bf16 rounding per output. */
typedef struct prefixlm_proj_gemm_args {
  const void* x;
  const void* w;
  void* y;
  int64_t x_stride, w_stride, y_stride;
  int32_t M, K, N;
  int32_t swiglu;
  int32_t norm;
  float eps;
  float* rstd;                   /* [M] fp32, written when norm != 0 */
} prefixlm_proj_gemm_args;
int prefixlm_proj_gemm(const prefixlm_proj_gemm_args* args, void* stream);

/* KV-cache attention, the inference path of the reference's attention layer
 * (flash_attn_with_kvcache, models/layers.py:147-151, simple_inference_engine.py:105-112).
 * The new rows k, v [B, S, H, D] are written into k_cache, v_cache [B, Smax, H, D] at rows
 * len_b .. len_b+S-1 (len_b = cache_seqlens[b], or cache_seqlen when cache_seqlens is
 * NULL; rows past Smax are dropped), then query i of row b attends the first
 * lk = min(Smax, len_b + S) cache keys (lk = min(Smax, len_b) without new rows), with
 * is_causal only keys j <= lk - S + i (bottom-right aligned). out: bf16 [B, S, H, D].
 * A call with cache_seqlens NULL and cache_seqlen 0 (the reference's prefill) runs the
 * varlen forward kernels over the new rows; every other call runs a split-K decode
 * kernel. All tensors have unit stride over D and element strides (batch, seq, head). */
typedef struct prefixlm_kvcache_args {
  const void* q;
  const void* k;                 /* new rows, or NULL (k and v together): attend the cache only */
  const void* v;
  void* k_cache;
  void* v_cache;
  void* out;
  int64_t q_stride_b, q_stride_s, q_stride_h;
  int64_t k_stride_b, k_stride_s, k_stride_h;
  int64_t v_stride_b, v_stride_s, v_stride_h;
  int64_t k_cache_stride_b, k_cache_stride_s, k_cache_stride_h;
  int64_t v_cache_stride_b, v_cache_stride_s, v_cache_stride_h;
  int64_t out_stride_b, out_stride_s, out_stride_h;
  const int32_t* cache_seqlens;  /* device int32 [B], or NULL */
  int32_t cache_seqlen;          /* used when cache_seqlens is NULL */
  int32_t batch;                 /* B */
  int32_t seqlen_q;              /* S */
  int32_t num_heads;             /* H */
  int32_t head_dim;              /* 128 */
  int32_t max_seqlen_cache;      /* Smax */
  int32_t is_causal;
  float softmax_scale;
  void* workspace;               /* >= prefixlm_kvcache_workspace_size(...) bytes */
  size_t workspace_bytes;
} prefixlm_kvcache_args;
size_t prefixlm_kvcache_workspace_size(int32_t batch, int32_t seqlen_q, int32_t num_heads, int32_t head_dim,
                                       int32_t max_seqlen_cache);
int prefixlm_kvcache_fwd(const prefixlm_kvcache_args* args, void* stream);

/* Synchronizes `stream` and reports the metadata error word the last call on this
 * workspace recorded (0 = consistent). Returns PREFIXLM_ERR_METADATA if it is nonzero.
 * The reference asserts instead (models/flash_attention_prefixlm_v2.py:103,169). */
int prefixlm_check_workspace(const void* workspace, void* stream, int32_t* error_word);

/* Message for the last nonzero status returned on this thread. */
const char* prefixlm_last_error(void);

/* Library version, e.g. 300 = 0.3.0 (PREFIXLM_VERSION). The minor version changes with
 * the layout of any buffer or argument struct the caller allocates: 0.2 stores out_lo as
 * int8 codes (0.1: bf16); 0.3 adds struct_size to the argument structs, ds_blocks to the
 * backward's, and stores only the attended dS blocks (with their bases in the plan). A
 * caller that sizes these buffers must check it before the first call. */
#define PREFIXLM_VERSION 300
int32_t prefixlm_version(void);

/* Per-kernel timing with HIP events recorded around each launch on its stream
 * (measurement aid; no counterpart in the reference). The timer is caller-owned state:
 * create one, pass it in the `timer` field of the args of the calls to time, read it,
 * destroy it. A timer must not be used by two threads at once. Kernel ids:
 * 0 fwd work list, 1 fwd, 2 fwd padding, 3 bwd work lists, 4 bwd pre-pass (delta),
 * 5 bwd dK/dV, 6 bwd padding, 7 bwd dQ. */
#define PREFIXLM_NUM_KERNELS 8
void* prefixlm_timer_create(void);          /* NULL if out of host memory */
void prefixlm_timer_destroy(void* timer);
/* Synchronizes on the timer's recorded events, writes total milliseconds and launch
 * counts per kernel id into the two arrays (length PREFIXLM_NUM_KERNELS) and clears the
 * records. */
int prefixlm_timer_read(void* timer, float* total_ms, int32_t* launches);

#ifdef __cplusplus
}
#endif

#endif  /* PREFIXLM_H_ */
