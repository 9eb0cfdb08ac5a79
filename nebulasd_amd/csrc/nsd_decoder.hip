// Decoder-stack executor for decode/verify rows (host code).
//
// nsd_decoder_forward enqueues, for every layer, the reference's layer body
// (swiftLLM/swiftllm/worker/layers/transformer_layer.py:83-201) on the
// caller's stream, all of it this library's kernels: fused add-RMSNorm, the
// q/k/v projection, the QK-norm + RoPE + KV-store prologue and paged
// attention (one launch, nsd_paged_attention_fused, for decode batches), the
// O projection, fused add-RMSNorm,
// fused up/gate + SiLU-and-mul and the down projection.  The layer loop runs
// in C++, so a layer costs the host its kernel enqueues and nothing else.
//
// The q/k/v, O and down projections are nsd_linear_partials calls: each
// writes fp32 split partials that the kernel after it sums where it reads
// the projection (the prologue, the post-attention add-RMSNorm, the next
// layer's input add-RMSNorm), so no launch only adds splits; after the last
// layer nsd_sum_partials writes the stack's output.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <new>
#include <vector>

#include "nsd_common.h"
#include "nsd_decoder.h"

using namespace nsd;

namespace {
constexpr int kMaxDecoderRows = 128;  // rows the fused up/gate kernel and the projections serve in one pass
}  // namespace

struct nsd_decoder {
  int layers = 0, hidden = 0, inter = 0, hq = 0, hkv = 0, d = 0, max_rows = 0;
  float eps = 0.f;
  int s_qkv = 0, s_o = 0, s_down = 0;  // split counts of the three projections
  std::vector<nsd_decoder_layer> w;
  // activations for max_rows rows
  float* part = nullptr;  // split partials of the projection in flight
  void* q = nullptr;      // [rows, hq, d]
  void* o = nullptr;      // [rows, hq d]
  void* oo = nullptr;     // [rows, hidden]
  void* h = nullptr;      // [rows, inter]

  ~nsd_decoder() {
    for (void* p : {(void*)part, q, o, oo, h})
      if (p) (void)hipFree(p);
  }
};

extern "C" int nsd_decoder_create(int num_layers, int hidden, int inter, int num_q_heads, int num_kv_heads,
                                  int head_dim, float rms_eps, const nsd_decoder_layer* layers, int max_rows,
                                  nsd_decoder** out) {
  if (out == nullptr || layers == nullptr) return fail(NSD_ERR_INVALID, "decoder_create: null pointer");
  *out = nullptr;
  if (num_layers < 1 || hidden < 128 || hidden % 128 || hidden > 8192 || inter < 128 || inter % 128 ||
      num_q_heads < 1 || num_kv_heads < 1 || num_q_heads % num_kv_heads)
    return fail(NSD_ERR_INVALID, "decoder_create: bad shape (layers %d, hidden %d, inter %d, heads %d/%d)",
                num_layers, hidden, inter, num_q_heads, num_kv_heads);
  if (head_dim != 128) return fail(NSD_ERR_UNSUPPORTED, "decoder_create: head_dim=%d (only 128)", head_dim);
  if (max_rows < 1 || max_rows > kMaxDecoderRows)
    return fail(NSD_ERR_UNSUPPORTED, "decoder_create: max_rows=%d outside [1, %d]", max_rows, kMaxDecoderRows);
  for (int i = 0; i < num_layers; ++i) {
    const nsd_decoder_layer& l = layers[i];
    if (!l.w_qkv || !l.w_o || !l.w_up_gate || !l.w_down || !l.norm_in || !l.norm_post)
      return fail(NSD_ERR_INVALID, "decoder_create: layer %d has a null weight", i);
    for (const void* p : {l.w_qkv, l.w_o, l.w_up_gate, l.w_down, l.norm_in, l.norm_post})
      if (!aligned16(p)) return fail(NSD_ERR_UNSUPPORTED, "decoder_create: layer %d weight not 16-byte aligned", i);
  }
  nsd_decoder* dec = new (std::nothrow) nsd_decoder();
  if (dec == nullptr) return fail(NSD_ERR_INVALID, "decoder_create: out of host memory");
  dec->layers = num_layers;
  dec->hidden = hidden;
  dec->inter = inter;
  dec->hq = num_q_heads;
  dec->hkv = num_kv_heads;
  dec->d = head_dim;
  dec->eps = rms_eps;
  dec->max_rows = max_rows;
  dec->w.assign(layers, layers + num_layers);
  const int64_t qkv_w = (int64_t)(num_q_heads + 2 * num_kv_heads) * head_dim;
  const int64_t r = max_rows;
  int rc = nsd_linear_splits(r, qkv_w, hidden, &dec->s_qkv);
  if (rc == NSD_OK) rc = nsd_linear_splits(r, hidden, (int64_t)num_q_heads * head_dim, &dec->s_o);
  if (rc == NSD_OK) rc = nsd_linear_splits(r, hidden, inter, &dec->s_down);
  if (rc != NSD_OK) {
    delete dec;
    return rc;
  }
  const int64_t part_elems = r * std::max({dec->s_qkv * qkv_w, (int64_t)dec->s_o * hidden,
                                           (int64_t)dec->s_down * hidden});
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&dec->part), part_elems * 4);
  if (e == hipSuccess) e = hipMalloc(&dec->q, r * num_q_heads * head_dim * 2);
  if (e == hipSuccess) e = hipMalloc(&dec->o, r * num_q_heads * head_dim * 2);
  if (e == hipSuccess) e = hipMalloc(&dec->oo, r * hidden * 2);
  if (e == hipSuccess) e = hipMalloc(&dec->h, r * inter * 2);
  if (e != hipSuccess) {
    delete dec;
    return fail(NSD_ERR_HIP, "decoder_create: %s", hipGetErrorString(e));
  }
  *out = dec;
  return NSD_OK;
}

extern "C" int nsd_decoder_destroy(nsd_decoder* dec) {
  delete dec;
  return NSD_OK;
}

extern "C" int nsd_decoder_forward(nsd_decoder* dec, void* x, void* residual, int64_t n_rows, void* k_cache,
                                   void* v_cache, int64_t num_blocks, const int32_t* block_table, int64_t bt_rows,
                                   int64_t bt_stride, const int32_t* seq_ids, const int32_t* seq_lens,
                                   const void* cos_cache, const void* sin_cache, int64_t n_positions,
                                   const int32_t* plan_host, const int32_t* plan_dev, void* attn_workspace,
                                   int64_t attn_workspace_bytes, float softmax_scale, int probe_layer,
                                   void* probe_q, void* probe_o, float* probe_lse, int32_t* status, void* stream) {
  if (dec == nullptr || x == nullptr || residual == nullptr)
    return fail(NSD_ERR_INVALID, "decoder_forward: null pointer");
  if (n_rows < 1 || n_rows > dec->max_rows)
    return fail(NSD_ERR_INVALID, "decoder_forward: n_rows=%lld outside [1, %d]", (long long)n_rows, dec->max_rows);
  if (!aligned16(x) || !aligned16(residual))
    return fail(NSD_ERR_UNSUPPORTED, "decoder_forward: x and residual must be 16-byte aligned");
  if (probe_layer >= dec->layers || (probe_layer >= 0 && (!probe_q || !probe_o || !probe_lse)))
    return fail(NSD_ERR_INVALID, "decoder_forward: probe layer %d of %d (or a null probe buffer)", probe_layer,
                dec->layers);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t H = dec->hidden, I = dec->inter, hq = dec->hq, hkv = dec->hkv, d = dec->d;
  const int64_t qkv_w = (hq + 2 * hkv) * d;
  // The prologue runs inside the attention's launch (one launch instead of
  // two, the same bits) where the plan keeps every sequence's rows in one
  // verify group and a group's query rows per kv head fit one 16-row tile
  // (decode batches: the Qwen3-0.6B draft layer 91.5 us against 93.8 us).
  // Past one tile every piece builds its group's query rows from the q/k/v
  // projection's five split partials, which gains nothing over the
  // prologue's own launch (the Qwen3-8B verify layer, 16 x 5 rows: 154.9 us
  // fused against 155.0 us), so verify batches keep two launches.  The
  // probe layer keeps the two calls, whose q it copies out.
  const bool fused = plan_host != nullptr && plan_host[kPlanRowsMax] <= 16 && plan_keeps_sequences_whole(plan_host);
  int rc = NSD_OK;
  for (int li = 0; li < dec->layers && rc == NSD_OK; ++li) {
    const nsd_decoder_layer& lw = dec->w[li];
    // input norm: over the embeddings for layer 0, else over the previous
    // layer's down projection (its partials)
    rc = li == 0 ? nsd_fused_add_rmsnorm_inplace(x, residual, lw.norm_in, n_rows, H, dec->eps, stream)
                 : nsd_fused_add_rmsnorm_partials(dec->part, dec->s_down, x, residual, lw.norm_in, n_rows, H,
                                                  dec->eps, stream);
    if (rc == NSD_OK) rc = nsd_linear_partials(x, lw.w_qkv, dec->part, n_rows, qkv_w, H, stream);
    const bool one_launch = fused && li != probe_layer;
    if (rc == NSD_OK && one_launch)
      rc = nsd_paged_attention_fused(nullptr, 0, nullptr, 0, nullptr, 0, dec->part, dec->s_qkv, lw.q_norm, lw.k_norm,
                                     dec->eps, cos_cache, sin_cache, n_positions, dec->o, nullptr, k_cache, v_cache,
                                     num_blocks, dec->layers, li, (int)hq, (int)hkv, (int)d, 16, block_table, bt_rows,
                                     bt_stride, plan_host, plan_dev, attn_workspace, attn_workspace_bytes,
                                     softmax_scale, status, stream);
    if (rc == NSD_OK && !one_launch)
      rc = nsd_qk_norm_rope_store_partials(dec->part, dec->s_qkv, dec->q, lw.q_norm, lw.k_norm, dec->eps, cos_cache,
                                           sin_cache, n_positions, k_cache, v_cache, block_table, bt_rows, bt_stride,
                                           seq_ids, seq_lens, n_rows, num_blocks, dec->layers, li, (int)hq, (int)hkv,
                                           (int)d, 16, status, stream);
    if (rc == NSD_OK && !one_launch)
      rc = nsd_paged_attention(dec->q, dec->o, li == probe_layer ? probe_lse : nullptr, k_cache, v_cache, num_blocks,
                               dec->layers, li, (int)hq, (int)hkv, (int)d, 16, block_table, bt_rows, bt_stride,
                               plan_host, plan_dev, attn_workspace, attn_workspace_bytes, softmax_scale, status,
                               stream);
    if (rc == NSD_OK && li == probe_layer) {
      const size_t bytes = (size_t)(n_rows * hq * d * 2);
      hipError_t e = hipMemcpyAsync(probe_q, dec->q, bytes, hipMemcpyDeviceToDevice, s);
      if (e == hipSuccess) e = hipMemcpyAsync(probe_o, dec->o, bytes, hipMemcpyDeviceToDevice, s);
      if (e != hipSuccess) rc = fail(NSD_ERR_HIP, "decoder_forward: probe copy: %s", hipGetErrorString(e));
    }
    if (rc == NSD_OK) rc = nsd_linear_partials(dec->o, lw.w_o, dec->part, n_rows, H, hq * d, stream);
    if (rc == NSD_OK)
      rc = nsd_fused_add_rmsnorm_partials(dec->part, dec->s_o, dec->oo, residual, lw.norm_post, n_rows, H, dec->eps,
                                          stream);
    if (rc == NSD_OK) rc = nsd_up_gate_silu_and_mul(dec->oo, lw.w_up_gate, dec->h, n_rows, H, I, stream);
    if (rc == NSD_OK) rc = nsd_linear_partials(dec->h, lw.w_down, dec->part, n_rows, H, I, stream);
  }
  if (rc == NSD_OK) rc = nsd_sum_partials(dec->part, dec->s_down, x, n_rows, H, stream);
  return rc;
}
