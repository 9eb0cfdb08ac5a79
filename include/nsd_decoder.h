/*
 * nsd_decoder.h -- C ABI of the decoder-stack executor for decode/verify rows.
 *
 * One call runs every layer of the reference's decoder for the decode and
 * verify rows of a forward: the loop over layers of
 * swiftLLM/swiftllm/worker/model.py:280-289 with the body of
 * LlamaTransformerLayer.forward (swiftLLM/swiftllm/worker/layers/
 * transformer_layer.py:83-201):
 *
 *   fused_add_rmsnorm(x, residual, input_layernorm)            (:98-103)
 *   qkv = x . W_qkv^T  (the q/k/v projections stacked; one GEMM for :107-109)
 *   QK-RMSNorm + RoPE + KV store of the new rows                (:114-145)
 *   o = paged_attention(q)                                       (:169-183)
 *     (these two in one launch, nsd_paged_attention_fused, for decode
 *     batches: a group's query rows per kv head within one 16-row tile and
 *     every sequence in one group; else two launches)
 *   o = o . W_o^T                                                (:189)
 *   fused_add_rmsnorm(o, residual, post_attention_layernorm)     (:192)
 *   h = fp16(up) * fp16(silu(fp16(gate))) of o . W_up_gate^T     (:199-200)
 *   x = h . W_down^T                                             (:201)
 *
 * on this library's kernels (nsd_attn.h), the q/k/v, O and down projections
 * included (nsd_linear_partials, whose split partials the next kernel sums
 * where it reads the projection), all enqueued on the caller's stream from
 * C++: the host cost of a layer is its kernel launches instead of a dozen
 * Python calls.  The embedding lookup before the stack and the final residual add
 * and post-layer after it stay with the caller.
 *
 * nsd_decoder_create allocates the executor's device buffers (activations
 * and projection partials for up to max_rows rows) and keeps the layer
 * weight pointers, which must stay valid until nsd_decoder_destroy.
 * nsd_decoder_forward allocates nothing and never synchronises the host; a
 * decoder serves one stream at a time (its activation buffers are shared
 * by its calls).
 */
#ifndef NSD_DECODER_H
#define NSD_DECODER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct nsd_decoder nsd_decoder;

/* One layer's weights, fp16 row-major device buffers (swiftLLM's
 * LlamaTransformerLayerWeight, swiftLLM/swiftllm/worker/weight.py:59-153,
 * with q/k/v stacked). */
typedef struct nsd_decoder_layer {
  const void* w_qkv;      /* [(Hq + 2 * Hkv) * d, hidden]: q rows, then k, then v */
  const void* w_o;        /* [hidden, Hq * d] */
  const void* w_up_gate;  /* [2 * inter, hidden]: up rows, then gate rows */
  const void* w_down;     /* [hidden, inter] */
  const void* norm_in;    /* [hidden] input_layernorm */
  const void* norm_post;  /* [hidden] post_attention_layernorm */
  const void* q_norm;     /* [d] q RMSNorm weight, or NULL */
  const void* k_norm;     /* [d] k RMSNorm weight, or NULL */
} nsd_decoder_layer;

/* hidden a multiple of 128 (<= 8192), inter a multiple of 128, head_dim 128,
 * num_q_heads a multiple of num_kv_heads, 1 <= max_rows <= 128. */
int nsd_decoder_create(int num_layers, int hidden, int inter, int num_q_heads, int num_kv_heads,
                       int head_dim, float rms_eps, const nsd_decoder_layer* layers, int max_rows,
                       nsd_decoder** out);

int nsd_decoder_destroy(nsd_decoder* dec);

/*
 * All layers for n_rows decode/verify rows (1 <= n_rows <= max_rows).
 * x [n_rows, hidden]: the embeddings on entry, the last layer's output on
 * return (the caller adds `residual` for the final hidden state, model.py:
 * 292).  residual [n_rows, hidden] must be zero on entry.  The caches,
 * block table, seq_ids / seq_lens (int32 device [n_rows]), cos/sin tables
 * and the attention plan and workspace are those of nsd_qk_norm_rope_store
 * and nsd_paged_attention for the same rows (the plan built from these
 * seq_ids / seq_lens).  probe_layer >= 0 copies that layer's attention input
 * q and output o ([n_rows, Hq, d] each) to probe_q / probe_o and writes its
 * natural-log LSE [n_rows, Hq] to probe_lse (for checks); that layer runs
 * the prologue and the attention as two launches (same results).  -1 for
 * none.  status: optional device int32 word (NSD_STATUS_*).
 */
int nsd_decoder_forward(nsd_decoder* dec, void* x, void* residual, int64_t n_rows,
                        void* k_cache, void* v_cache, int64_t num_blocks,
                        const int32_t* block_table, int64_t bt_rows, int64_t bt_stride,
                        const int32_t* seq_ids, const int32_t* seq_lens,
                        const void* cos_cache, const void* sin_cache, int64_t n_positions,
                        const int32_t* plan_host, const int32_t* plan_dev, void* attn_workspace,
                        int64_t attn_workspace_bytes, float softmax_scale, int probe_layer,
                        void* probe_q, void* probe_o, float* probe_lse, int32_t* status,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NSD_DECODER_H */
