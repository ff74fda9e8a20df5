/*
 * ataraxos_attn.h — C ABI of the MI355X (gfx950) attention library
 * `libataraxos_attn.so`.
 *
 * The library holds the GPU side of the attention hot path of the ataraxos
 * transformer networks (Move, Setup and Belief networks).  It has no libtorch
 * dependency: every tensor crosses this boundary as a raw device pointer plus
 * element strides, and every call is an asynchronous launch on the caller's
 * HIP stream.
 *
 * Conventions shared by every entry point
 *   - Return value: ATX_OK (0) on success, a negative ATX_ERR_* code on
 *     failure.  No C++ exception crosses the boundary.  The text of the most
 *     recent failure on the calling thread is available from atx_last_error().
 *   - Memory: the caller allocates every buffer (inputs and outputs).  The
 *     library allocates no device memory and keeps no mutable global state,
 *     so calls are re-entrant and may run concurrently on different streams.
 *   - Strides are in ELEMENTS, not bytes.  The innermost (head_dim / feature)
 *     dimension must be contiguous (stride 1) and every row must start on a
 *     16-byte boundary.
 *   - `stream` is a hipStream_t passed as void* (NULL = the legacy default
 *     stream).  Nothing synchronises with the host.
 *   - Argument validation happens on the host before any HIP call, so invalid
 *     arguments are reported without touching a GPU.
 */
#ifndef ATARAXOS_ATTN_H
#define ATARAXOS_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ATX_ABI_VERSION 3

/* Return codes. */
#define ATX_OK 0
#define ATX_ERR_INVALID_ARGUMENT (-1) /* null pointer, bad size or stride */
#define ATX_ERR_UNSUPPORTED (-2)      /* valid, but outside the kernels' range */
#define ATX_ERR_LAUNCH (-3)           /* the HIP runtime rejected the launch */
#define ATX_ERR_ABI (-4)              /* params struct from another ABI version */

/* Element types. */
#define ATX_DTYPE_FP32 0
#define ATX_DTYPE_BF16 1
#define ATX_DTYPE_FP16 2

/* ------------------------------------------------------------------------ */
/* Fused attention forward                                                  */
/* ------------------------------------------------------------------------ */

/*
 * O[b, s, h, :] = softmax_j( scale * Q[b, s, h, :] . K[b, j, h / G, :]
 *                            + mask[b, s, j] ) . V[b, j, h / G, :]
 * with G = num_heads / num_kv_heads (grouped-query attention) and mask = -inf
 * where the key is padded out (key_pad[b, j] != 0) or, if `causal`, where
 * j > s (top-left alignment, as torch.triu(ones(S_q, S_kv), 1)).
 * A query row whose keys are all masked produces NaN, as a softmax over an
 * all -inf row does.
 *
 * Q, K, V and O are BSHD tensors ([batch, seq, heads, head_dim], head_dim
 * contiguous) given by base pointer and element strides; the Q/K/V views the
 * reference takes of its [B, S, E] projection outputs are accepted as they
 * are.  O is written in the same dtype as the inputs.
 */
typedef struct AtxAttnParams {
    int32_t abi_version; /* must equal ATX_ABI_VERSION */
    int32_t dtype;       /* ATX_DTYPE_*: Q, K, V and O all have this type */
    int32_t batch;
    int32_t seq_q;
    int32_t seq_kv;
    int32_t num_heads;    /* query heads H */
    int32_t num_kv_heads; /* H_kv, divides H */
    int32_t head_dim;     /* D */
    const void* q;
    int64_t q_stride_b, q_stride_s, q_stride_h;
    const void* k;
    int64_t k_stride_b, k_stride_s, k_stride_h;
    const void* v;
    int64_t v_stride_b, v_stride_s, v_stride_h;
    void* o;
    int64_t o_stride_b, o_stride_s, o_stride_h;
    float scale;             /* > 0; the reference uses 1/sqrt(D) */
    int32_t causal;          /* nonzero: mask j > s */
    const uint8_t* key_pad;  /* optional [batch, seq_kv]; nonzero = ignore key */
    int64_t key_pad_stride_b;
    /* Attention dropout (training; attention.py:312-313 and FA2's
     * dropout_p, :236-253): each softmax weight (b, h, i, j) is zeroed with
     * probability dropout_p and the survivors scaled by 1 / (1 - dropout_p).
     * The keep decision is a hash of the element's flat index
     * ((b * H + h) * seq_q + i) * seq_kv + j and (dropout_seed,
     * dropout_offset); atx_dropout_mask writes the same decisions, and
     * atx_attn_bwd given the same three values differentiates through them.
     * 0 <= dropout_p < 1; dropout_p > 0 needs head_dim 48 or 64. */
    float dropout_p;
    int32_t reserved_dropout; /* 0 */
    uint64_t dropout_seed;
    uint64_t dropout_offset;
} AtxAttnParams;

/*
 * Replaces the backend dispatch of MultiHeadAttention.forward and the four
 * backend bodies it selects between:
 *   stratego/networks/attention.py:192-200  (dispatch)
 *   stratego/networks/attention.py:222-234  (_forward_fa3)
 *   stratego/networks/attention.py:236-253  (_forward_fa2, dropout_p = 0)
 *   stratego/networks/attention.py:255-279  (_forward_sdpa)
 *   stratego/networks/attention.py:281-316  (_forward_math, the semantics)
 * and the GQA expansion of stratego/networks/attention.py:210-220.
 * The key-padding mask serves the Belief decoder's cross-attention
 * (memory_key_padding_mask = ~hidden_mask, stratego/networks/belief_net.py:159).
 *
 * Supported range: dtype BF16, FP16 or FP32; head_dim a multiple of 16 up to
 * 128; 1 <= seq_kv <= 256; any seq_q >= 1 and batch >= 1.
 */
int atx_attn_fwd(const AtxAttnParams* params, void* stream);

/* Gradients of atx_attn_fwd: given Q, K, V, the forward output O and dO, write
 * dQ ([B, S_q, H, D]), dK and dV ([B, S_kv, H_kv, D]). */
typedef struct AtxAttnBwdParams {
    int32_t abi_version; /* must equal ATX_ABI_VERSION */
    int32_t dtype;       /* ATX_DTYPE_BF16, FP16 or FP32: every tensor has this type */
    int32_t batch;
    int32_t seq_q;
    int32_t seq_kv;
    int32_t num_heads;    /* H */
    int32_t num_kv_heads; /* H_kv, divides H */
    int32_t head_dim;     /* D */
    const void* q;
    int64_t q_stride_b, q_stride_s, q_stride_h;
    const void* k;
    int64_t k_stride_b, k_stride_s, k_stride_h;
    const void* v;
    int64_t v_stride_b, v_stride_s, v_stride_h;
    const void* o;
    int64_t o_stride_b, o_stride_s, o_stride_h;
    const void* d_o;
    int64_t do_stride_b, do_stride_s, do_stride_h;
    void* dq;
    int64_t dq_stride_b, dq_stride_s, dq_stride_h;
    void* dk;
    int64_t dk_stride_b, dk_stride_s, dk_stride_h;
    void* dv;
    int64_t dv_stride_b, dv_stride_s, dv_stride_h;
    float scale;
    int32_t causal;
    const uint8_t* key_pad; /* optional [batch, seq_kv]; nonzero = ignore key */
    int64_t key_pad_stride_b;
    /* The forward's dropout (see AtxAttnParams): the same dropout_p,
     * dropout_seed and dropout_offset, and o the forward's output with it. */
    float dropout_p;
    int32_t reserved_dropout; /* 0 */
    uint64_t dropout_seed;
    uint64_t dropout_offset;
} AtxAttnBwdParams;

/*
 * Replaces the autograd backward of the attention the reference trains
 * through (stratego/training/move_trainer.py:140 -> MultiHeadAttention.forward,
 * stratego/networks/attention.py:281-316 on the math path, or FA3 / FA2 /
 * SDPA's own backward).  The softmax is recomputed from Q and K.
 *
 * With G = num_heads / num_kv_heads > 1 (grouped-query attention), dK and dV
 * of KV head j sum the gradients of query heads j*G .. j*G + G - 1, the
 * gradient of the repeat_interleave of stratego/networks/attention.py:210-220.
 *
 * Supported range: BF16 / FP16 / FP32 (FP32: full fp32 products); head_dim a
 * multiple of 16 up to 128; 1 <= seq_kv <= 256; 1 <= seq_q <= 2^20 (query
 * rows are staged in blocks when they do not fit in LDS at once); FP32 with
 * head_dim >= 80 only up to 128 keys.  Gradients of key padded or causally
 * masked entries are zero; a query row with no usable key gets dQ = 0 and
 * makes its (batch, head)'s dV NaN, as autograd through a softmax over an
 * all -inf row does.
 */
int atx_attn_bwd(const AtxAttnBwdParams* params, void* stream);

/*
 * keep[b, h, i, j] = 1 where attention dropout with (p, seed, offset) keeps
 * weight (b, h, i, j) of a [batch, num_heads, seq_q, seq_kv] attention, else
 * 0: the decisions atx_attn_fwd / atx_attn_bwd make.  `keep` is a contiguous
 * uint8 device buffer of batch * num_heads * seq_q * seq_kv bytes.
 * Asynchronous on `stream`.  No counterpart in the reference (its math path
 * returns no mask; FA2 returns one only in debug mode): for checking a
 * dropout run against an explicit mask.
 */
int atx_dropout_mask(int32_t batch, int32_t num_heads, int32_t seq_q, int32_t seq_kv, float p, uint64_t seed,
                     uint64_t offset, uint8_t* keep, void* stream);

/* ------------------------------------------------------------------------ */
/* Key-query policy head: logits + legal-move mask (+ softmax)              */
/* ------------------------------------------------------------------------ */

#define ATX_KQ_OUT_PROBS 0  /* softmax over all S*S entries, illegal = 0.0 */
#define ATX_KQ_OUT_LOGITS 1 /* scaled logits, illegal = -1e10 */

/*
 * For every sample b, L[i, j] = scale * q[b, i, :] . k[b, j, :] over
 * i, j < seq ("from" square i, "to" square j).  Entries whose mask byte is
 * zero are illegal.  The output is fp32 [batch, seq * seq] in from-major
 * order (index i * seq + j):
 *   ATX_KQ_OUT_LOGITS: L, with illegal entries set to -1e10;
 *   ATX_KQ_OUT_PROBS:  softmax of that over all seq*seq entries; illegal
 *                      entries are exactly 0.0.  A sample with no legal
 *                      entry gets the uniform 1/(seq*seq), which is what the
 *                      softmax of an all -1e10 row gives.
 * `mask` may be NULL (every entry legal).
 */
typedef struct AtxKqParams {
    int32_t abi_version;
    int32_t dtype; /* of q and k: ATX_DTYPE_BF16, FP16 or FP32 */
    int32_t batch;
    int32_t seq;   /* squares per sample, 1..128 */
    int32_t dim;   /* policy_d_model, a multiple of 8 */
    int32_t out_mode; /* ATX_KQ_OUT_* */
    const void* q;
    int64_t q_stride_b, q_stride_s;
    const void* k;
    int64_t k_stride_b, k_stride_s;
    const uint8_t* mask; /* optional [batch, seq, seq]; nonzero = legal */
    int64_t mask_stride_b, mask_stride_s;
    float* out; /* [batch, seq * seq], contiguous per sample */
    int64_t out_stride_b;
    float scale; /* > 0; the reference divides by sqrt(policy_d_model) */
} AtxKqParams;

/*
 * Replaces KeyQueryPolicyHead's logit product and mask,
 *   stratego/networks/move_net.py:92-95,
 * and (ATX_KQ_OUT_PROBS) the softmax its callers apply to the result:
 *   stratego/training/selfplay.py:284, stratego/training/move_trainer.py:118,
 *   stratego/search/rollouts.py:82, stratego/search/mirror_descent.py:126.
 */
int atx_kq_masked_softmax_fwd(const AtxKqParams* params, void* stream);

/*
 * Backward of the policy head: for every sample b, given the upstream
 * gradient G = grad[b] (fp32, [seq * seq] from-major) with respect to the
 * forward's output,
 *   ATX_KQ_OUT_LOGITS: dL = G on legal entries, 0 on illegal ones;
 *   ATX_KQ_OUT_PROBS:  dL = P * (G - sum(G * P)) on legal entries, 0 on
 *                      illegal ones, with P = probs[b] the forward's output;
 * then dq[b] = scale * dL k[b] and dk[b] = scale * dL^T q[b] (dL as
 * [seq, seq]), written in q's dtype.  Masked entries get no gradient, as
 * through masked_fill; a sample with no legal entry gets dq = dk = 0.
 * q / k in BF16, FP16 or FP32 (FP32: fp32 products, the precision the
 * reference trains in).  dim a multiple of 16 up to 128, or of 64 up to 4096
 * (the reference's policy_d_model = 384, stratego/networks/move_net.py:151);
 * FP32: a multiple of 16 up to 4096.
 */
typedef struct AtxKqBwdParams {
    int32_t abi_version;
    int32_t dtype;    /* of q, k, dq, dk: ATX_DTYPE_BF16, FP16 or FP32 */
    int32_t batch;
    int32_t seq;      /* 1..128 */
    int32_t dim;      /* see above */
    int32_t out_mode; /* ATX_KQ_OUT_*: what `grad` is the gradient of */
    const void* q;
    int64_t q_stride_b, q_stride_s;
    const void* k;
    int64_t k_stride_b, k_stride_s;
    const uint8_t* mask; /* optional [batch, seq, seq]; nonzero = legal */
    int64_t mask_stride_b, mask_stride_s;
    const float* grad;   /* [batch, seq * seq], contiguous per sample */
    int64_t grad_stride_b;
    const float* probs;  /* ATX_KQ_OUT_PROBS: the forward's output; else NULL */
    int64_t probs_stride_b;
    void* dq;
    int64_t dq_stride_b, dq_stride_s;
    void* dk;
    int64_t dk_stride_b, dk_stride_s;
    float scale;
} AtxKqBwdParams;

/*
 * Replaces the autograd backward through KeyQueryPolicyHead's product and
 * mask (stratego/networks/move_net.py:92-95), and for ATX_KQ_OUT_PROBS the
 * caller's softmax, that the Move trainer's loss.backward() runs
 * (stratego/training/move_trainer.py:115-140).
 */
int atx_kq_bwd(const AtxKqBwdParams* params, void* stream);

/* ------------------------------------------------------------------------ */
/* Fused self-attention layer: projections + attention + output projection  */
/* ------------------------------------------------------------------------ */

/*
 * For every sample b (x, y: [batch, seq, embed_dim], rows contiguous):
 *   q = x Wq^T + bq, k = x Wk^T + bk, v = x Wv^T + bv   (rounded to dtype)
 *   o = per head softmax(scale * q_h k_h^T [+ top-left causal mask]) v_h
 *                                                        (rounded to dtype)
 *   y = o Wo^T + bo
 * with W* the nn.Linear weights [embed_dim, embed_dim] (out x in,
 * contiguous) and b* optional biases [embed_dim] (NULL = none).
 * head_dim 64 (embed_dim = 64 * num_heads), num_heads in {2, 4, 6, 8},
 * seq <= 128 within 160 KiB of LDS (embed_dim 512: seq <= 112), 16-bit only.
 */
typedef struct AtxMhaParams {
    int32_t abi_version;
    int32_t dtype; /* ATX_DTYPE_BF16 or FP16: x, weights, biases and y */
    int32_t batch;
    int32_t seq;
    int32_t embed_dim;
    int32_t num_heads;
    int32_t causal;
    int32_t reserved; /* 0 */
    const void* x;
    int64_t x_stride_b, x_stride_s;
    const void* w_q;
    const void* w_k;
    const void* w_v;
    const void* w_o;
    const void* b_q; /* optional */
    const void* b_k;
    const void* b_v;
    const void* b_o;
    void* y;
    int64_t y_stride_b, y_stride_s;
    float scale; /* the reference uses 1 / sqrt(head_dim) */
    /* The attention half of a pre-LN block, y = x + layer(LayerNorm(x))
     * (stratego/networks/transformer.py:143 with dropout inactive): with
     * ln_weight set, each x row is normalised (fp32 mean and biased
     * variance, eps ln_eps, then * ln_weight + ln_bias, rounded to dtype)
     * before the projections; with residual = 1 the layer output, rounded to
     * dtype, is added to x and rounded again.  y may be x itself.  Both
     * need the persistent form's shape (6 heads of 64, 65 <= seq <= 101);
     * elsewhere they are refused with ATX_ERR_UNSUPPORTED.  NULL / 0: off. */
    const void* ln_weight; /* [embed_dim], dtype; NULL: no LayerNorm */
    const void* ln_bias;   /* [embed_dim], dtype; NULL: zero */
    float ln_eps;
    int32_t residual;
} AtxMhaParams;

/*
 * Replaces MultiHeadAttention.forward for self-attention
 * (stratego/networks/attention.py:152-204 with key_value = None): the
 * q/k/v projections (:175-179), the backend dispatch (:192-200) and the
 * output projection (:203-204), in one launch.
 */
int atx_mha_fwd(const AtxMhaParams* params, void* stream);

/*
 * The same layer with w_q, w_k, w_v and w_o in the packed tile order that
 * atx_mha_pack_weight writes (everything else as atx_mha_fwd; identical
 * results).  The kernel's weight loads then read whole cache lines: at the
 * Move-network shape this is ~10 % faster, at 40-64 positions up to 2x.
 * The weights are those of attention.py:113-116 (q/k/v/out_proj), packed
 * once per weight update by the caller; the reference has no counterpart.
 */
int atx_mha_fwd_packed(const AtxMhaParams* params, void* stream);

/*
 * packed = w [dim, dim] (nn.Linear weight, out x in, contiguous, 16-bit
 * dtype) in the packed tile order: for row tile rt = 0 .. dim/16 - 1 and
 * k-step kt = 0 .. dim/32 - 1, 64 chunks of 8 elements, chunk 16 g + m
 * holding w[16 rt + m, 32 kt + 8 g .. 32 kt + 8 g + 7], at element offset
 * ((rt * (dim / 32) + kt) * 64 + 16 g + m) * 8.  dim a multiple of 32 up to
 * 4096; w and packed 16-byte aligned and not overlapping.  Asynchronous on
 * `stream`.
 */
int atx_mha_pack_weight(int32_t dtype, int32_t dim, const void* w, void* packed, void* stream);

/* Bytes of the workspace atx_mha_fwd_ws needs at this embed_dim: the four
 * weights in the packed tile order, 4 * embed_dim^2 * 2 (0 if embed_dim < 1). */
int64_t atx_mha_workspace_bytes(int32_t embed_dim);

/*
 * atx_mha_fwd with the weights in the nn.Linear order (as atx_mha_fwd takes
 * them), run through the packed-order kernel: one launch rearranges all four
 * weights into `workspace` (the layout of atx_mha_pack_weight, q, k, v, out
 * consecutively), a second runs the layer from there.  Results are identical
 * to atx_mha_fwd and atx_mha_fwd_packed.  `workspace`: device memory of at
 * least atx_mha_workspace_bytes(embed_dim) bytes, 256-byte aligned, not
 * overlapping x, y or a weight; its contents are overwritten.  Because the
 * weights are rearranged on every call, an in-place change of a weight
 * (optimizer step, EMA swap through param.data.copy_) is always seen.
 * Replaces the same reference lines as atx_mha_fwd
 * (stratego/networks/attention.py:152-204 with key_value = None).
 */
int atx_mha_fwd_ws(const AtxMhaParams* params, void* workspace, int64_t workspace_bytes, void* stream);

/* Size of the device array behind atx_mha_fwd_noalloc: the four packed
 * weights at embed_dim 512 (4 * 512 * 512 * 2 bytes). */
#define ATX_MHA_NOALLOC_SCRATCH_BYTES (2 * 1024 * 1024)

/*
 * atx_mha_fwd_ws without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The weights are rearranged into a library-owned device array of
 * ATX_MHA_NOALLOC_SCRATCH_BYTES (one per GPU, held until the process ends),
 * so embed_dim <= 512; a larger layer is refused with ATX_ERR_UNSUPPORTED.
 * The call allocates nothing: its first call on a device looks up that
 * device's array (hipGetSymbolAddress), every call launches the weight
 * rearrangement and the layer on `stream`, which must belong to the current
 * device.  Results are identical to atx_mha_fwd_ws and atx_mha_fwd.
 * Every call on one GPU shares that GPU's array: calls whose executions
 * overlap on one GPU (different streams, or graphs replayed concurrently)
 * race on it; calls ordered on one stream do not.
 */
int atx_mha_fwd_noalloc(const AtxMhaParams* params, void* stream);

/* ------------------------------------------------------------------------ */
/* Single-query attention over a KV cache (incremental decode)              */
/* ------------------------------------------------------------------------ */

/*
 * o[b, h, :] = softmax_{j < n_b}(scale * q[b, h, :] . K[b, h / G, j, :])
 *              . V[b, h / G, j, :]
 * with n_b = kv_lens[b] when kv_lens is given, else kv_len.  The cache rows
 * are K[b, g, j, :] = k_cache + b*k_stride_b + g*k_stride_h + j*k_stride_s.
 * When k_new / v_new are given ([batch, num_kv_heads, head_dim]), row n_b - 1
 * is taken from them AND written into the cache, so one call appends the
 * newest token and attends over it.  The result equals the last row of a full
 * causal recompute over n_b tokens.
 */
typedef struct AtxDecodeParams {
    int32_t abi_version;
    int32_t dtype; /* ATX_DTYPE_BF16, FP16 or FP32, for every tensor */
    int32_t batch;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t head_dim; /* a multiple of 8, up to 256 */
    int32_t kv_capacity; /* rows allocated per cache head; lengths are clamped to it */
    int32_t kv_len;   /* used when kv_lens is NULL; 1 <= kv_len <= kv_capacity */
    const int32_t* kv_lens; /* optional device array [batch]; a length < 1 yields NaN */
    const void* q;
    int64_t q_stride_b, q_stride_h;
    void* k_cache;
    int64_t k_stride_b, k_stride_h, k_stride_s;
    void* v_cache;
    int64_t v_stride_b, v_stride_h, v_stride_s;
    const void* k_new; /* optional, with v_new */
    int64_t k_new_stride_b, k_new_stride_h;
    const void* v_new;
    int64_t v_new_stride_b, v_new_stride_h;
    void* o;
    int64_t o_stride_b, o_stride_h;
    float scale;
} AtxDecodeParams;

/*
 * No one-call counterpart in the reference: SetupNetwork re-runs its causal
 * MultiHeadAttention over the whole prefix for every placed piece
 * (stratego/training/selfplay.py:139-146,181 -> stratego/networks/
 * setup_net.py:117 -> stratego/networks/attention.py:281-316 with
 * is_causal = True).  This entry point returns the last row of that
 * recompute from a KV cache.
 */
int atx_attn_decode_fwd(const AtxDecodeParams* params, void* stream);

/* ------------------------------------------------------------------------ */
/* Library information                                                      */
/* ------------------------------------------------------------------------ */

/* Text of the last failure on the calling thread ("" if none). */
const char* atx_last_error(void);

/* ATX_ABI_VERSION of the built library. */
int atx_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ATARAXOS_ATTN_H */
