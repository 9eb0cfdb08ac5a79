// Decoder-stack executor for decode/verify rows (host code).
//
// nsd_decoder_forward enqueues, for every layer, the reference's layer body
// (swiftLLM/swiftllm/worker/layers/transformer_layer.py:83-201) on the
// caller's stream: this library's fused add-RMSNorm, strided QK-norm + RoPE +
// KV-store prologue, paged attention and fused up/gate + SiLU-and-mul, and
// hipBLASLt GEMMs for the q/k/v, O and down projections.  The layer loop
// runs in C++, so a layer costs the host a dozen enqueues.
//
// GEMMs: y[M, N] = x[M, K] . W[N, K]^T with row-major fp16 x, W and y is,
// in hipBLASLt's column-major terms, y^T (N x M, ld N) = op_T(W^T stored
// K x N, ld K) . (x^T stored K x M, ld K), fp32 accumulation: the
// computation F.linear hands to the same library.  The matrix layouts and
// the heuristic's first algorithm are cached per (M, N, K).
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <new>
#include <tuple>
#include <vector>

#include "nsd_common.h"
#include "nsd_decoder.h"

using namespace nsd;

namespace {

constexpr int64_t kGemmWorkspace = 32ll << 20;
constexpr int kMaxDecoderRows = 128;  // rows the fused up/gate kernel serves in one pass

struct Gemm {
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

const char* lt_error(hipblasStatus_t s) {
  switch (s) {
    case HIPBLAS_STATUS_SUCCESS: return "success";
    case HIPBLAS_STATUS_NOT_INITIALIZED: return "not initialized";
    case HIPBLAS_STATUS_ALLOC_FAILED: return "allocation failed";
    case HIPBLAS_STATUS_INVALID_VALUE: return "invalid value";
    case HIPBLAS_STATUS_MAPPING_ERROR: return "mapping error";
    case HIPBLAS_STATUS_EXECUTION_FAILED: return "execution failed";
    case HIPBLAS_STATUS_INTERNAL_ERROR: return "internal error";
    case HIPBLAS_STATUS_NOT_SUPPORTED: return "not supported";
    default: return "error";
  }
}

}  // namespace

struct nsd_decoder {
  int layers = 0, hidden = 0, inter = 0, hq = 0, hkv = 0, d = 0, max_rows = 0;
  float eps = 0.f;
  std::vector<nsd_decoder_layer> w;
  hipblasLtHandle_t lt = nullptr;
  hipblasLtMatmulDesc_t mm = nullptr;
  void* gemm_ws = nullptr;
  std::map<std::tuple<int64_t, int64_t, int64_t>, Gemm> gemms;
  std::mutex mu;  // the GEMM cache
  // activations for max_rows rows
  void* qkv = nullptr;  // [rows, (hq + 2 hkv) d]
  void* q = nullptr;    // [rows, hq, d]
  void* o = nullptr;    // [rows, hq d]
  void* oo = nullptr;   // [rows, hidden]
  void* h = nullptr;    // [rows, inter]

  ~nsd_decoder() {
    for (auto& kv : gemms) {
      hipblasLtMatrixLayoutDestroy(kv.second.a);
      hipblasLtMatrixLayoutDestroy(kv.second.b);
      hipblasLtMatrixLayoutDestroy(kv.second.c);
    }
    if (mm) hipblasLtMatmulDescDestroy(mm);
    if (lt) hipblasLtDestroy(lt);
    for (void* p : {gemm_ws, qkv, q, o, oo, h})
      if (p) (void)hipFree(p);
  }

  // y[M, N] = x[M, K] . w[N, K]^T on stream s.
  int gemm(const void* x, const void* wt, void* y, int64_t M, int64_t N, int64_t K, hipStream_t s) {
    const Gemm* g = nullptr;
    {
      std::lock_guard<std::mutex> lock(mu);
      auto key = std::make_tuple(M, N, K);
      auto it = gemms.find(key);
      if (it == gemms.end()) {
        Gemm e;
        hipblasStatus_t st = hipblasLtMatrixLayoutCreate(&e.a, HIP_R_16F, K, N, K);
        if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&e.b, HIP_R_16F, K, M, K);
        if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&e.c, HIP_R_16F, N, M, N);
        hipblasLtMatmulPreference_t pref = nullptr;
        if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatmulPreferenceCreate(&pref);
        uint64_t ws = kGemmWorkspace;
        if (st == HIPBLAS_STATUS_SUCCESS)
          st = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                                     sizeof(ws));
        hipblasLtMatmulHeuristicResult_t res[1];
        int found = 0;
        if (st == HIPBLAS_STATUS_SUCCESS)
          st = hipblasLtMatmulAlgoGetHeuristic(lt, mm, e.a, e.b, e.c, e.c, pref, 1, res, &found);
        if (pref) hipblasLtMatmulPreferenceDestroy(pref);
        if (st != HIPBLAS_STATUS_SUCCESS || found < 1 || res[0].workspaceSize > (size_t)kGemmWorkspace) {
          for (auto l : {e.a, e.b, e.c})
            if (l) hipblasLtMatrixLayoutDestroy(l);
          return fail(NSD_ERR_HIP, "decoder: no hipBLASLt algorithm for %lld x %lld x %lld (%s)", (long long)M,
                      (long long)N, (long long)K, st != HIPBLAS_STATUS_SUCCESS ? lt_error(st) : "none found");
        }
        e.algo = res[0].algo;
        it = gemms.emplace(key, e).first;
      }
      g = &it->second;
    }
    const float alpha = 1.f, beta = 0.f;
    const hipblasStatus_t st = hipblasLtMatmul(lt, mm, &alpha, wt, g->a, x, g->b, &beta, y, g->c, y, g->c, &g->algo,
                                               gemm_ws, kGemmWorkspace, s);
    if (st != HIPBLAS_STATUS_SUCCESS)
      return fail(NSD_ERR_HIP, "decoder: hipblasLtMatmul %lld x %lld x %lld: %s", (long long)M, (long long)N,
                  (long long)K, lt_error(st));
    return NSD_OK;
  }
};

extern "C" int nsd_decoder_create(int num_layers, int hidden, int inter, int num_q_heads, int num_kv_heads,
                                  int head_dim, float rms_eps, const nsd_decoder_layer* layers, int max_rows,
                                  nsd_decoder** out) {
  if (out == nullptr || layers == nullptr) return fail(NSD_ERR_INVALID, "decoder_create: null pointer");
  *out = nullptr;
  if (num_layers < 1 || hidden < 128 || hidden % 128 || hidden > 8192 || inter < 16 || inter % 16 ||
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
  hipblasStatus_t st = hipblasLtCreate(&dec->lt);
  if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatmulDescCreate(&dec->mm, HIPBLAS_COMPUTE_32F, HIP_R_32F);
  const int32_t op_t = HIPBLAS_OP_T, op_n = HIPBLAS_OP_N;
  if (st == HIPBLAS_STATUS_SUCCESS)
    st = hipblasLtMatmulDescSetAttribute(dec->mm, HIPBLASLT_MATMUL_DESC_TRANSA, &op_t, sizeof(op_t));
  if (st == HIPBLAS_STATUS_SUCCESS)
    st = hipblasLtMatmulDescSetAttribute(dec->mm, HIPBLASLT_MATMUL_DESC_TRANSB, &op_n, sizeof(op_n));
  if (st != HIPBLAS_STATUS_SUCCESS) {
    delete dec;
    return fail(NSD_ERR_HIP, "decoder_create: hipBLASLt set-up: %s", lt_error(st));
  }
  const int64_t qkv_w = (int64_t)(num_q_heads + 2 * num_kv_heads) * head_dim;
  const int64_t r = max_rows;
  hipError_t e = hipMalloc(&dec->gemm_ws, kGemmWorkspace);
  if (e == hipSuccess) e = hipMalloc(&dec->qkv, r * qkv_w * 2);
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
  auto* qkv = static_cast<char*>(dec->qkv);
  int rc = NSD_OK;
  for (int li = 0; li < dec->layers && rc == NSD_OK; ++li) {
    const nsd_decoder_layer& lw = dec->w[li];
    rc = nsd_fused_add_rmsnorm_inplace(x, residual, lw.norm_in, n_rows, H, dec->eps, stream);
    if (rc == NSD_OK) rc = dec->gemm(x, lw.w_qkv, dec->qkv, n_rows, qkv_w, H, s);
    if (rc == NSD_OK)
      rc = nsd_qk_norm_rope_store_strided(qkv, qkv_w, dec->q, qkv + hq * d * 2, qkv_w, qkv + (hq + hkv) * d * 2,
                                          qkv_w, lw.q_norm, lw.k_norm, dec->eps, cos_cache, sin_cache, n_positions,
                                          k_cache, v_cache, block_table, bt_rows, bt_stride, seq_ids, seq_lens,
                                          n_rows, num_blocks, dec->layers, li, (int)hq, (int)hkv, (int)d, 16, status,
                                          stream);
    if (rc == NSD_OK)
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
    if (rc == NSD_OK) rc = dec->gemm(dec->o, lw.w_o, dec->oo, n_rows, H, hq * d, s);
    if (rc == NSD_OK) rc = nsd_fused_add_rmsnorm_inplace(dec->oo, residual, lw.norm_post, n_rows, H, dec->eps, stream);
    if (rc == NSD_OK) rc = nsd_up_gate_silu_and_mul(dec->oo, lw.w_up_gate, dec->h, n_rows, H, I, stream);
    if (rc == NSD_OK) rc = dec->gemm(dec->h, lw.w_down, x, n_rows, H, I, s);
  }
  return rc;
}
